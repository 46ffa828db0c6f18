#!/usr/bin/env python3
"""Build oracle/_ref/libref_scalar.so from the reference's own scalar format functions.

Checker infrastructure only (never the product).  The reference's qwen_moe_q3k.c cannot be
compiled here as a whole (it includes riscv_vector.h and carries RISC-V inline asm), but the
functions that define the block formats and quantizers are plain C.  This recipe reads that file
where it lies, copies the definitions named in DEFS (found by their declarations, the braces of a
function matched to its end) into a temporary directory, compiles them there together with
oracle/ref_scalar_driver.c (wrappers of our own) and writes only the shared libraries into
oracle/_ref/ (libref_scalar.so with floating-point contraction off, libref_scalar_fma.so with
a*b - c fused).  The temporary copy is deleted; nothing of the reference's text enters the
repository.  Each definition's line range is printed, so the citations can be checked.

clang is used because the block structs hold _Float16 fields (gcc 11 has no _Float16 on x86).

Usage: python3 oracle/ref_scalar.py [/root/reference]
"""
import os
import re
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "_ref", "libref_scalar.so")
OUT_FMA = os.path.join(HERE, "_ref", "libref_scalar_fma.so")
SRC = "qwen_moe_q3k.c"

# (kind, name) in dependency order; kind "typedef" = `typedef struct {...} name;`,
# "fn" = a function definition.
DEFS = [
    ("typedef", "TInfo"), ("typedef", "Gguf"),
    ("fn", "f16f"), ("fn", "f32_to_f16"), ("fn", "f16_to_f32"),
    ("typedef", "q8_0_native"), ("fn", "quantize_q8_0_native"), ("fn", "pack_A_i8"),
    ("typedef", "block_q3_K"), ("typedef", "block_q5_K"),
    ("fn", "q5k_get_scale_min"), ("fn", "dequantize_q5_K_block"), ("fn", "dequantize_q3_K_block"),
    ("fn", "pack_A_q3k"), ("fn", "gguf_dequant_into"),
]


def line_of(text, pos):
    return text.count("\n", 0, pos) + 1


def find_typedef(text, name):
    m = re.search(r"typedef\s+struct\s*\{[^{}]*\}\s*" + re.escape(name) + r"\s*;", text)
    if not m:
        raise SystemExit("typedef %s not found in %s" % (name, SRC))
    return m.start(), m.end()


def find_fn(text, name):
    m = re.search(r"^static\s+(?:inline\s+)?[A-Za-z_][\w\s\*]*?\b" + re.escape(name) + r"\s*\([^;{]*\)\s*\{",
                  text, flags=re.M)
    if not m:
        raise SystemExit("function %s not found in %s" % (name, SRC))
    depth, i = 0, m.end() - 1
    while True:
        c = text[i]
        if c == "{":
            depth += 1
        elif c == "}":
            depth -= 1
            if depth == 0:
                return m.start(), i + 1
        i += 1


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    path = os.path.join(ref, SRC)
    if not os.path.exists(path):
        raise SystemExit("reference source %s not present: nothing to build" % path)
    text = open(path).read()
    parts = []
    for kind, name in DEFS:
        a, b = (find_typedef if kind == "typedef" else find_fn)(text, name)
        print("%s:%d-%d  %s %s" % (SRC, line_of(text, a), line_of(text, b), kind, name))
        parts.append(text[a:b])
    cc = shutil.which("clang") or "/opt/rocm/llvm/bin/clang"
    os.makedirs(os.path.dirname(OUT), exist_ok=True)
    tmp = tempfile.mkdtemp(prefix="ref_scalar_")
    try:
        src = os.path.join(tmp, "ref_fns.c")
        with open(src, "w") as f:
            f.write("\n\n".join(parts) + "\n")
        # Two builds: -ffp-contract=off rounds every float expression as written (the oracle is built
        # the same way); the second lets the compiler fuse a*b - c into one FMA, as the reference's
        # own gcc -O3 builds for riscv64 may (GCC's default contraction for GNU C).
        for out, flags in ((OUT, ["-ffp-contract=off"]), (OUT_FMA, ["-ffp-contract=fast", "-mfma"])):
            cmd = [cc, "-O2", "-std=gnu11", "-fPIC", "-shared", "-fvisibility=hidden", "-w"] + flags + \
                  ['-DREF_SCALAR_SRC="%s"' % src, os.path.join(HERE, "ref_scalar_driver.c"), "-o", out + ".tmp", "-lm"]
            subprocess.run(cmd, check=True)
            os.replace(out + ".tmp", out)
            print("built", out)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


if __name__ == "__main__":
    main()
