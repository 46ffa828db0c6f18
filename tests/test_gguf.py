"""GGUF reader of libx100hip (include/x100_gguf.h) on synthetic files written by gguf.write, checked
against the bytes written and against the reference's own bench/gguf_dump.c, built unmodified into
oracle/_ref by oracle/Makefile (the listings must agree byte for byte).  Host-only: no GPU."""
import os
import struct
import subprocess

import numpy as np
import pytest

import gguf
import synth
import x100hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_DUMP = os.path.join(ROOT, "oracle", "_ref", "gguf_dump")


def qwen_like(n_layers=1, d=512, ff=256, n_exp=8, vocab=300, n_head=4, n_kv=2, hd=128):
    """Key/values and tensors shaped like a (small) Qwen3-MoE checkpoint, in its mixed precision."""
    kv = [
        ("general.architecture", gguf.STRING, "qwen3moe"),
        ("general.name", gguf.STRING, "synthetic"),
        ("qwen3moe.block_count", gguf.U32, n_layers),
        ("qwen3moe.context_length", gguf.U32, 40960),
        ("qwen3moe.embedding_length", gguf.U32, d),
        ("qwen3moe.feed_forward_length", gguf.U32, 6144),
        ("qwen3moe.attention.head_count", gguf.U32, n_head),
        ("qwen3moe.attention.head_count_kv", gguf.U32, n_kv),
        ("qwen3moe.rope.freq_base", gguf.F32, 1000000.0),
        ("qwen3moe.attention.layer_norm_rms_epsilon", gguf.F32, 1e-6),
        ("qwen3moe.expert_used_count", gguf.U32, 4),
        ("qwen3moe.attention.key_length", gguf.U32, hd),
        ("qwen3moe.attention.value_length", gguf.I32, hd),
        ("qwen3moe.expert_count", gguf.U32, n_exp),
        ("qwen3moe.expert_feed_forward_length", gguf.U32, ff),
        ("tokenizer.ggml.model", gguf.STRING, "gpt2"),
        ("tokenizer.ggml.tokens", gguf.ARRAY, (gguf.STRING, ["tok%d" % i for i in range(vocab)])),
        ("tokenizer.ggml.token_type", gguf.ARRAY, (gguf.I32, list(range(vocab)))),
        ("tokenizer.ggml.bos_token_id", gguf.U32, 151643),
        ("general.file_type", gguf.U32, 12),
        ("test.u8", gguf.U8, 200), ("test.i8", gguf.I8, -5), ("test.u16", gguf.U16, 65000),
        ("test.i16", gguf.I16, -30000), ("test.bool", gguf.BOOL, True), ("test.u64", gguf.U64, 2 ** 40),
        ("test.i64", gguf.I64, -(2 ** 40)), ("test.f64", gguf.F64, 2.5),
        ("test.nested", gguf.ARRAY, (gguf.ARRAY, [(gguf.U16, [1, 2, 3]), (gguf.STRING, ["a", "bc"])])),
        ("test.vocab_note", gguf.STRING, "x" * 300),
        ("test.expert_f64", gguf.F64, 0.125),
    ]
    ten = []

    def add(name, qt, dims, seed):
        if qt == gguf.F32_T:
            data = synth.normal_f32(seed, (int(np.prod(dims)),)).tobytes()
        elif qt == gguf.F16_T:
            data = synth.normal_f32(seed, (int(np.prod(dims)),)).astype(np.float16).tobytes()
        else:
            K = dims[0]
            rows = int(np.prod(dims[1:]))
            data = synth.quant_weight(qt, rows, K, seed).tobytes()
        ten.append((name, qt, dims, data))

    add("token_embd.weight", gguf.Q3_K, [d, vocab], 1)
    for l in range(n_layers):
        p = "blk.%d." % l
        add(p + "attn_norm.weight", gguf.F32_T, [d], 10 + l)
        add(p + "attn_q.weight", gguf.Q3_K, [d, n_head * hd], 11 + l)
        add(p + "attn_k.weight", gguf.Q8_0, [d, n_kv * hd], 12 + l)
        add(p + "attn_v.weight", gguf.Q4_0, [d, n_kv * hd], 13 + l)
        add(p + "attn_output.weight", gguf.Q5_K, [n_head * hd, d], 14 + l)
        add(p + "attn_q_norm.weight", gguf.F16_T, [hd], 15 + l)
        add(p + "ffn_gate_inp.weight", gguf.F32_T, [d, n_exp], 16 + l)
        add(p + "ffn_gate_exps.weight", gguf.Q4_K, [d, ff, n_exp], 17 + l)
        add(p + "ffn_up_exps.weight", gguf.Q4_K, [d, ff, n_exp], 18 + l)
        add(p + "ffn_down_exps.weight", gguf.Q4_K, [ff, d, n_exp], 19 + l)
    add("output_norm.weight", gguf.F32_T, [d], 98)
    add("output.weight", gguf.Q6_K, [d, vocab], 99)
    return kv, ten


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    path = str(tmp_path_factory.mktemp("gguf") / "m.gguf")
    kv, ten = qwen_like()
    offs = gguf.write(path, kv, ten)
    return path, kv, ten, offs


def test_parse_matches_what_was_written(model):
    path, kv, ten, offs = model
    with gguf.GGUF(path) as g:
        assert g.version == 3 and g.n_tensors == len(ten) and g.n_kv == len(kv) and g.alignment == 32
        assert g.data_offset % 32 == 0
        assert g.keys() == [k for k, _, _ in kv]
        for i, (name, qt, dims, data) in enumerate(ten):
            t = g.tensor(i)
            assert t.name.decode() == name and t.type == qt and t.shape == tuple(dims)
            assert t.offset == offs[i] and t.n_elems == int(np.prod(dims)) and t.n_bytes == len(data)
            assert t.array().tobytes() == data
            t2 = g.find(name)
            assert t2.data == t.data and t2.offset == t.offset
        assert not g.has("blk.7.attn_q.weight")
        with pytest.raises(x100hip.X100Error) as e:
            g.find("missing.weight")
        assert e.value.code == x100hip.X100_ENOTFOUND


def test_metadata_getters(model):
    path = model[0]
    with gguf.GGUF(path) as g:
        assert g.get_str("general.architecture") == "qwen3moe"
        assert g.get_int("qwen3moe.block_count") == 1 and g.get_int("qwen3moe.attention.value_length") == 128
        assert g.get_int("test.u8") == 200 and g.get_int("test.i8") == -5 and g.get_int("test.u16") == 65000
        assert g.get_int("test.i16") == -30000 and g.get_int("test.u64") == 2 ** 40
        assert g.get_int("test.i64") == -(2 ** 40)
        assert g.get_float("qwen3moe.rope.freq_base") == 1e6 and g.get_float("test.f64") == 2.5
        assert g.get_float("qwen3moe.attention.layer_norm_rms_epsilon") == float(np.float32(1e-6))
        assert g.get_arr_str("tokenizer.ggml.tokens", 0) == b"tok0"
        assert g.get_arr_str("tokenizer.ggml.tokens", 299) == b"tok299"
        key, typ, et, cnt = g.kv_at(g.keys().index("test.nested"))
        assert (typ, et, cnt) == (gguf.ARRAY, gguf.ARRAY, 2)
        for bad in (lambda: g.get_int("general.architecture"), lambda: g.get_str("test.u8"),
                    lambda: g.get_float("test.bool"), lambda: g.get_int("nope"),
                    lambda: g.get_arr_str("tokenizer.ggml.token_type", 0)):
            with pytest.raises(x100hip.X100Error) as e:
                bad()
            assert e.value.code == x100hip.X100_ENOTFOUND
        with pytest.raises(x100hip.X100Error) as e:
            g.get_arr_str("tokenizer.ggml.tokens", 300)
        assert e.value.code == x100hip.X100_EINVAL


def test_qwen3moe_params(model, tmp_path):
    with gguf.GGUF(model[0]) as g:
        p = g.qwen3moe()
    assert p == {"block_count": 1, "embd": 512, "ffn": 6144, "n_head": 4, "n_head_kv": 2, "head_dim": 128,
                 "vocab": 300, "n_exp": 8, "n_act": 4, "moe_ffn": 256, "rope_base": 1e6, "n_tokens": 300}
    # absent keys take gguf_open's defaults (qwen_moe.c:129)
    path = str(tmp_path / "bare.gguf")
    gguf.write(path, [("general.architecture", gguf.STRING, "qwen3moe")], [])
    with gguf.GGUF(path) as g:
        p = g.qwen3moe()
    assert (p["n_exp"], p["n_act"], p["moe_ffn"], p["rope_base"], p["vocab"], p["block_count"]) == \
        (128, 8, 768, 1e6, 0, 0)


def test_alignment_key(tmp_path):
    path = str(tmp_path / "a64.gguf")
    data = [("a", gguf.F32_T, [3], np.arange(3, dtype=np.float32).tobytes()),
            ("b", gguf.Q8_0, [64], synth.quant_weight(synth.Q8_0, 1, 64, 3).tobytes())]
    offs = gguf.write(path, [("general.alignment", gguf.U32, 64)], data, alignment=64)
    with gguf.GGUF(path) as g:
        assert g.alignment == 64 and g.data_offset % 64 == 0
        assert [g.tensor(i).offset for i in range(2)] == offs == [0, 64]
        assert g.find("b").array().tobytes() == data[1][3]


def test_block_geometry():
    for qt in (synth.Q4_0, synth.Q8_0, synth.Q3_K, synth.Q4_K, synth.Q5_K, synth.Q6_K):
        lib = x100hip.lib()
        assert lib.x100_gguf_block_bytes(qt) == synth.BLOCK_BYTES[qt]
        assert lib.x100_gguf_block_elems(qt) == synth.BLOCK_ELEMS[qt]
    assert gguf.type_name(12) == "Q4_K" and gguf.type_name(30) == "BF16" and gguf.type_name(31) == "?"
    assert gguf.type_name(4) == ""


@pytest.mark.skipif(not os.path.exists(REF_DUMP), reason="oracle/_ref/gguf_dump not built (make -C oracle)")
@pytest.mark.parametrize("grep", [None, "blk.0", "exps", "zzz", ""])
def test_listing_matches_reference_gguf_dump(model, grep):
    path = model[0]
    args = [REF_DUMP, path] + ([grep] if grep is not None else [])
    ref = subprocess.run(args, capture_output=True, check=True).stdout
    assert gguf.dump(path, grep) == ref


@pytest.mark.skipif(not os.path.exists(REF_DUMP), reason="oracle/_ref/gguf_dump not built (make -C oracle)")
def test_listing_matches_reference_many_layers(tmp_path):
    # 4 layers: 49 tensors, past the tool's 40-line limit without a grep
    path = str(tmp_path / "m4.gguf")
    kv, ten = qwen_like(n_layers=4, d=256, ff=256, n_exp=4, vocab=64, n_head=2, n_kv=1, hd=128)
    gguf.write(path, kv, ten)
    for grep in (None, "ffn"):
        args = [REF_DUMP, path] + ([grep] if grep else [])
        ref = subprocess.run(args, capture_output=True, check=True).stdout
        assert gguf.dump(path, grep) == ref
    out = subprocess.run(["python", os.path.join(ROOT, "x100-gemm_amd", "gguf.py"), path], capture_output=True,
                         check=True).stdout
    assert out == subprocess.run([REF_DUMP, path], capture_output=True, check=True).stdout


def open_code(path):
    try:
        gguf.GGUF(path).close()
        return x100hip.X100_OK
    except x100hip.X100Error as e:
        return e.code


def test_malformed_files(tmp_path, model):
    good = open(model[0], "rb").read()
    p = str(tmp_path / "bad.gguf")

    def code(blob):
        with open(p, "wb") as f:
            f.write(blob)
        return open_code(p)

    assert open_code(str(tmp_path / "absent.gguf")) == x100hip.X100_EIO
    assert code(b"") == x100hip.X100_EFORMAT
    assert code(b"GGUX" + good[4:]) == x100hip.X100_EFORMAT
    assert code(good[:4] + struct.pack("<I", 1) + good[8:]) == x100hip.X100_EFORMAT
    assert code(good[:4] + struct.pack("<I", 4) + good[8:]) == x100hip.X100_EFORMAT
    # absurd counts
    assert code(good[:8] + struct.pack("<Q", 1 << 60) + good[16:]) == x100hip.X100_EFORMAT
    assert code(good[:16] + struct.pack("<Q", 1 << 60) + good[24:]) == x100hip.X100_EFORMAT
    # every truncation of the file fails cleanly (the last tensor's data runs to the end)
    cuts = sorted(set(list(range(0, 2048, 7)) + list(range(len(good) - 2048, len(good), 97)) + [len(good) - 1]))
    for n in cuts:
        assert code(good[:n]) == x100hip.X100_EFORMAT, n
    assert code(good) == x100hip.X100_OK


def test_malformed_tensor_records(tmp_path):
    p = str(tmp_path / "t.gguf")

    def one(dims, qt=gguf.Q8_0, data=b"\0" * 34):
        gguf.write(p, [], [("w", qt, dims, data)])
        return open_code(p)

    assert one([32]) == x100hip.X100_OK
    assert one([1, 1, 1, 1, 32]) == x100hip.X100_EFORMAT          # more than 4 dims
    assert one([]) == x100hip.X100_EFORMAT                         # no dims
    assert one([33]) == x100hip.X100_EFORMAT                       # not a whole number of blocks
    assert one([64]) == x100hip.X100_EFORMAT                       # data runs past the end
    assert one([2 ** 40, 2 ** 40]) == x100hip.X100_EFORMAT         # byte count overflows
    assert one([32], qt=200) == x100hip.X100_OK                    # unknown type: listed, not loadable
    with gguf.GGUF(p) as g:
        t = g.find("w")
        assert t.n_bytes == 0 and not t.data and gguf.type_name(t.type) == "?"
