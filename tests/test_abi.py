"""The C-ABI library loads and exports exactly what include/*.h declares (no GPU calls)."""
import glob
import os
import re
import subprocess

import x100hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b([A-Za-z_]\w*)\s*\(", text, flags=re.M):
            name = m.group(1)
            if name not in ("if", "defined", "sizeof"):
                names.add(name)
    return names


def test_headers_declare_the_binding_exports():
    assert declared_functions() == set(x100hip.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = x100hip.lib()
    for name in declared_functions():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", x100hip.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    assert exported == declared_functions()


def test_library_does_not_link_the_oracle():
    out = subprocess.run(["nm", "-D", x100hip.LIB_PATH], capture_output=True, text=True, check=True).stdout
    assert "orc_" not in out and "gemm_ref_i8" not in out
    deps = subprocess.run(["readelf", "-d", x100hip.LIB_PATH], capture_output=True, text=True,
                          check=True).stdout
    assert "oracle" not in deps and "amdhip64" in deps


def test_pure_host_entry_points():
    # size helpers run on the host only
    assert x100hip.gguf_bytes(x100hip.Q4_0, 4096, 4096) == 4096 * 128 * 18
    assert x100hip.gguf_bytes(x100hip.Q4_K, 6144, 2048) == 6144 * 8 * 144
    assert x100hip.gguf_bytes(x100hip.Q3_K, 6144, 2048) == 6144 * 8 * 110
    assert x100hip.gguf_bytes(x100hip.Q4_K, 10, 100) == 0
    # K-quants: one section per super-block column, 148 (Q4_K) / 114 (Q3_K) bytes per row, each
    # section rounded up to 256 bytes
    assert x100hip.packed_bytes(x100hip.Q4_K, 6144, 2048) == 8 * 6144 * 148
    assert x100hip.packed_bytes(x100hip.Q3_K, 6144, 2048) == 8 * 6144 * 114
    assert x100hip.packed_bytes(x100hip.Q3_K, 5, 512) == 2 * 768
    assert x100hip.packed_bytes(x100hip.Q4_0, 4096, 4096) >= 4096 * 128 * 18
    assert x100hip.strerror(x100hip.X100_EINVAL).startswith("invalid")


def test_integration_snippet_is_the_compiled_code():
    """The integration guide's C code for the engine's Lin (lin_hip_new / lin_hip_mm) is compiled,
    verbatim, into x100-gemm_amd/host/x100_host.c (run by tests/test_host_gpu.py)."""
    doc = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    src = open(os.path.join(ROOT, "x100-gemm_amd", "host", "x100_host.c")).read()
    blocks = re.findall(r"```c\n(.*?)```", doc, flags=re.S)
    lin = [b for b in blocks if "lin_hip_new(LinHip" in b]
    assert len(lin) == 1
    body = "\n".join(l for l in lin[0].splitlines() if not l.startswith("#include")).strip()
    assert body in src
