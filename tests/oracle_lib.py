"""ctypes binding of oracle/liboracle.so -- the CPU restatement the parity tests compare against.

Test infrastructure only: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, never by the product path.
"""
import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_PATH = os.path.join(ROOT, "oracle", "liboracle.so")
REF_PATH = os.path.join(ROOT, "oracle", "_ref", "libx100ref.so")

Q4_0, Q8_0, Q3_K, Q4_K, Q5_K, Q6_K, Q8_K = 2, 8, 11, 12, 13, 14, 15
DT_Q8_0 = np.dtype([("d", "<u2"), ("qs", "i1", (32,))])
DT_Q8_K = np.dtype([("d", "<f4"), ("qs", "i1", (256,)), ("bsums", "<i2", (16,))])
DT_A_I8 = np.dtype([("s", "<f4"), ("asum", "<i2"), ("qs", "i1", (32,))])   # pack_A_i8 record
assert DT_Q8_0.itemsize == 34 and DT_Q8_K.itemsize == 292 and DT_A_I8.itemsize == 38

class LayerCfg(ctypes.Structure):
    """orc_layer_cfg."""
    _fields_ = [(n, ctypes.c_int) for n in ("d", "n_head", "n_head_kv", "head_dim", "ff", "n_exp", "n_act", "ctx")] + \
               [("eps", ctypes.c_float), ("rope_base", ctypes.c_float)] + \
               [(n, ctypes.c_int) for n in ("wq_type", "wk_type", "wv_type", "wo_type")]


_o = None
_r = None


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def oracle():
    global _o
    if _o is None:
        if not os.path.exists(ORACLE_PATH):
            raise FileNotFoundError("oracle/liboracle.so not built (make -C oracle)")
        L = ctypes.CDLL(ORACLE_PATH)
        i, p, f = ctypes.c_int, ctypes.c_void_p, ctypes.c_float
        L.orc_f32_to_f16.argtypes = [f]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f16_to_f32.restype = f
        L.gemm_ref_i8.argtypes = [i, i, i, p, p, p]
        L.gemm_ref_i8.restype = None
        L.orc_gemm_i8_mt.argtypes = [i, i, i, p, p, p, i]
        L.orc_gemm_i8_mt.restype = None
        L.orc_dequant_row.argtypes = [i, p, i, p]
        L.orc_quantize_q8_0.argtypes = [p, i, p]
        L.orc_quantize_q8_0.restype = None
        L.orc_quantize_q8_K.argtypes = [p, i, p]
        L.orc_quantize_q8_K.restype = None
        L.orc_quantize_q4_0.argtypes = [p, i, p]
        L.orc_quantize_q4_0.restype = None
        L.orc_quantize_i8.argtypes = [p, i, p]
        L.orc_quantize_i8.restype = None
        L.orc_requant_q8_0.argtypes = [i, i, i, p, p]
        L.orc_qgemv_q8w.argtypes = [i, i, i, p, p, p]
        L.orc_qgemv.argtypes = [i, i, i, i, p, p, p]
        L.orc_qgemv_q.argtypes = [i, i, i, i, p, p, p]
        L.orc_moe_layer.argtypes = [i, i, i, i, i, p, p, p, p, p, p, i, p, p]
        L.orc_moe_route.argtypes = [i, i, i, i, p, p, p, p, p]
        L.orc_gemv_int.argtypes = [i, i, i, p, p, p]
        L.orc_gemv_int.restype = None
        L.orc_pack_w_int4.argtypes = [i, i, p, p]
        L.orc_pack_w_int8.argtypes = [i, i, p, p]
        L.orc_rmsnorm.argtypes = [p, p, p, i, f]
        L.orc_rmsnorm.restype = None
        L.orc_rope_table.argtypes = [p, p, i, i, f]
        L.orc_rope_table.restype = None
        L.orc_rope_apply.argtypes = [p, i, p, p]
        L.orc_rope_apply.restype = None
        L.orc_attn_decode.argtypes = [ctypes.POINTER(LayerCfg)] + [p] * 9 + [i, p]
        L.orc_decode_layer.argtypes = [ctypes.POINTER(LayerCfg)] + [p] * 14 + [i, p, p, p]
        L.orc_swiglu.argtypes = [f, f]
        L.orc_swiglu.restype = f
        _o = L
    return _o


def reference():
    """The reference's own gemm_ref_i8 built from its sources (oracle/_ref), or None."""
    global _r
    if _r is None and os.path.exists(REF_PATH):
        L = ctypes.CDLL(REF_PATH)
        i, p = ctypes.c_int, ctypes.c_void_p
        L.gemm_ref_i8.argtypes = [i, i, i, p, p, p]
        L.gemm_ref_i8.restype = None
        _r = L
    return _r


def gemm_ref_i8(A, B, C, threads=1):
    """C += A.B (in place) with the oracle (threads > 1: row-parallel, same arithmetic)."""
    M, K = A.shape
    N = B.shape[1]
    A = np.ascontiguousarray(A)
    B = np.ascontiguousarray(B)
    assert C.dtype == np.int32 and C.flags.c_contiguous
    if threads > 1:
        oracle().orc_gemm_i8_mt(M, N, K, _p(A), _p(B), _p(C), threads)
    else:
        oracle().gemm_ref_i8(M, N, K, _p(A), _p(B), _p(C))
    return C


def dequant_row(qtype, blocks, K):
    out = np.empty(K, dtype=np.float32)
    b = np.ascontiguousarray(blocks)
    rc = oracle().orc_dequant_row(qtype, _p(b), K, _p(out))
    assert rc == 0
    return out


def quantize_q8_0(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.size // 32, dtype=DT_Q8_0)
    oracle().orc_quantize_q8_0(_p(x), x.size, _p(out))
    return out


def quantize_q8_K(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.size // 256, dtype=DT_Q8_K)
    oracle().orc_quantize_q8_K(_p(x), x.size, _p(out))
    return out


def quantize_i8(x):
    """pack_A_i8 records (fp32 scale, int16 sum, 32 int8) of one fp32 row."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.size // 32, dtype=DT_A_I8)
    oracle().orc_quantize_i8(_p(x), x.size, _p(out))
    return out


def requant_q8_0(qtype, W):
    """Load-time requantization of a Q8_0 / Q5_K / Q6_K weight (N rows of GGUF blocks) to
    N x K/32 Q8_0 blocks."""
    Wc = np.ascontiguousarray(W)
    N = Wc.shape[0]
    K = Wc.shape[1] * (32 if qtype == Q8_0 else 256)
    out = np.zeros((N, K // 32), dtype=DT_Q8_0)
    rc = oracle().orc_requant_q8_0(qtype, N, K, _p(Wc), _p(out))
    assert rc == 0
    return out


def qgemv_q8w(Wq8, x):
    """Per-call part of the int8 path for a weight already requantized by requant_q8_0."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    N = Wq8.shape[0]
    y = np.empty((M, N), dtype=np.float32)
    rc = oracle().orc_qgemv_q8w(M, N, K, _p(np.ascontiguousarray(Wq8)), _p(x), _p(y))
    assert rc == 0
    return y


def quantize_q4_0(w, dtype):
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.zeros(w.size // 32, dtype=dtype)
    oracle().orc_quantize_q4_0(_p(w), w.size, _p(out))
    return out


def qgemv(qtype, W, x):
    """y (M x N) for GGUF blocks W (N rows) and fp32 x (M x K)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    N = W.shape[0]
    y = np.empty((M, N), dtype=np.float32)
    Wc = np.ascontiguousarray(W)
    rc = oracle().orc_qgemv(qtype, M, N, K, _p(Wc), _p(x), _p(y))
    assert rc == 0
    return y


def moe_layer(hn, R, Wg, Wu, Wd, n_act, out=None, residual=False):
    hn = np.ascontiguousarray(hn, dtype=np.float32)
    M, d = hn.shape
    n_exp = R.shape[0]
    ff = Wg.shape[1]
    if out is None:
        out = np.zeros((M, d), dtype=np.float32)
    sel = np.zeros((M, n_act), dtype=np.int32)
    sw = np.zeros((M, n_act), dtype=np.float32)
    R = np.ascontiguousarray(R, dtype=np.float32)
    rc = oracle().orc_moe_layer(M, d, ff, n_exp, n_act, _p(hn), _p(R), _p(np.ascontiguousarray(Wg)),
                                _p(np.ascontiguousarray(Wu)), _p(np.ascontiguousarray(Wd)), _p(out),
                                1 if residual else 0, _p(sel), _p(sw))
    assert rc == 0
    return out, sel, sw


def moe_route(hn, R, n_act):
    hn = np.ascontiguousarray(hn, dtype=np.float32)
    M, d = hn.shape
    n_exp = R.shape[0]
    logits = np.zeros((M, n_exp), dtype=np.float32)
    sel = np.zeros((M, n_act), dtype=np.int32)
    sw = np.zeros((M, n_act), dtype=np.float32)
    rc = oracle().orc_moe_route(M, d, n_exp, n_act, _p(hn), _p(np.ascontiguousarray(R, dtype=np.float32)),
                                _p(logits), _p(sel), _p(sw))
    assert rc == 0
    return logits, sel, sw


def gemv_int(W, x):
    """y[M][N] = W[N][K] . x[M][K]^T (int32 exact), bench/q4_gemv.c:101-103."""
    W = np.ascontiguousarray(W, dtype=np.int8)
    x = np.ascontiguousarray(x, dtype=np.int8)
    N, K = W.shape
    M = x.shape[0]
    y = np.zeros((M, N), np.int32)
    oracle().orc_gemv_int(M, N, K, _p(W), _p(x), _p(y))
    return y


def pack_w(int4, W):
    """Packed tile layout of pack_w_int4 / pack_w_int8 (bench/q4_gemv.c:37-62)."""
    W = np.ascontiguousarray(W, dtype=np.int8)
    N, K = W.shape
    if int4:
        out = np.zeros(N * K // 2, np.uint8)
        rc = oracle().orc_pack_w_int4(N, K, _p(W), _p(out))
    else:
        out = np.zeros(N * K, np.int8)
        rc = oracle().orc_pack_w_int8(N, K, _p(W), _p(out))
    assert rc == 0
    return out


def rmsnorm(x, w, eps):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.empty_like(x)
    oracle().orc_rmsnorm(_p(out), _p(x), _p(w), x.size, eps)
    return out


def rope_table(hd, pos, base):
    c = np.empty(hd // 2, np.float32)
    s_ = np.empty(hd // 2, np.float32)
    oracle().orc_rope_table(_p(c), _p(s_), hd, pos, base)
    return c, s_


def _a(x):
    return None if x is None else _p(np.ascontiguousarray(x))


def attn_decode(cfg, L, kc, vc, pos, h):
    """h (modified in place) += attention; kc / vc (modified in place) get k, v at pos.  L: dict of
    numpy weights (GGUF blocks for wq / wk / wv / wo)."""
    assert h.dtype == np.float32 and h.flags.c_contiguous and kc.flags.c_contiguous and vc.flags.c_contiguous
    rc = oracle().orc_attn_decode(ctypes.byref(cfg), _a(L["attn_norm"]), _a(L["q_norm"]), _a(L["k_norm"]),
                                  _a(L["wq"]), _a(L["wk"]), _a(L["wv"]), _a(L["wo"]), _p(kc), _p(vc), pos, _p(h))
    assert rc == 0


def decode_layer(cfg, L, kc, vc, pos, h):
    assert h.dtype == np.float32 and h.flags.c_contiguous
    sel = np.zeros(cfg.n_act, np.int32)
    sw = np.zeros(cfg.n_act, np.float32)
    rc = oracle().orc_decode_layer(ctypes.byref(cfg), _a(L["attn_norm"]), _a(L["q_norm"]), _a(L["k_norm"]),
                                   _a(L["wq"]), _a(L["wk"]), _a(L["wv"]), _a(L["wo"]), _a(L["ffn_norm"]),
                                   _a(L["router"]), _a(L["wg"]), _a(L["wu"]), _a(L["wd"]), _p(kc), _p(vc), pos, _p(h),
                                   _p(sel), _p(sw))
    assert rc == 0
    return sel, sw

