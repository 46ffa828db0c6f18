"""ctypes binding of libx100hip.so (the C ABI declared in include/x100_*.h).

Thin host-side mirror used by the tests, bench.py and smoke(): every call goes straight to the
gfx950 kernels through the C entry points; there is no CPU fallback.  Device memory and streams
come from the caller (torch tensors are convenient: pass tensor.data_ptr() and
torch.cuda.current_stream().cuda_stream).

Entry points and what they replace in the reference:
  gemm_ime_i8 / gemm_hip_i8 / gemm_hip_i8_dev   include/x100_gemm.h:60-61 (C += A*B, int8->int32)
  qgemv_hip (+ x100q_pack)                      lin_mm of qwen_moe.c:101-107 on Q4_0/Q4_K/Q3_K;
                                                lin_mm_i8_x of qwen_moe_q3k.c:1075 on Q8_0/Q5_K/Q6_K
  moe_layer_hip / moe_layer_hip_ws              the MoE block of qwen_moe.c:294-311 (library or
                                                caller scratch); moe_pack_experts: load-time
                                                regrouping of the expert tensors (tiled=True)
  gemv_int4_hip / gemv_int8_hip (+ packers)     gemv_nb_int4 / gemv_nb_int8 of bench/q4_gemv.c:67-99
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libx100hip.so")

Q4_0, Q8_0, Q3_K, Q4_K, Q5_K, Q6_K = 2, 8, 11, 12, 13, 14

X100_OK, X100_EINVAL, X100_ENODEV, X100_EHIP, X100_ENOMEM = 0, -1, -2, -3, -4
X100_EIO, X100_EFORMAT, X100_ENOTFOUND, X100_ESCRATCH = -5, -6, -7, -8
MOE_NOALLOC_MAX_BYTES = 8 << 20

# Every symbol declared in include/x100_gemm.h, x100_gemv_tile.h, x100_qgemv.h, x100_moe.h,
# x100_gguf.h, x100_decode.h.
EXPORTS = (
    "gemm_ime_i8", "gemm_hip_i8", "gemm_hip_i8_dev", "gemm_hip_i8_dev_set", "gemm_hip_i8_dev_variant",
    "x100_hip_detect", "x100_hip_caps_print", "x100_hip_strerror",
    "x100_tile_bytes", "x100_pack_w_int4", "x100_pack_w_int8", "gemv_int4_hip", "gemv_int8_hip",
    "x100q_gguf_bytes", "x100q_packed_bytes", "x100q_pack", "qgemv_hip", "x100q_check_quant_div",
    "moe_layer_hip", "moe_layer_workspace_bytes", "moe_layer_hip_ws", "moe_layer_hip_noalloc",
    "moe_pack_experts",
    "x100_gguf_open", "x100_gguf_close", "x100_gguf_version", "x100_gguf_n_tensors", "x100_gguf_n_kv",
    "x100_gguf_alignment", "x100_gguf_data_offset", "x100_gguf_tensor_at", "x100_gguf_find",
    "x100_gguf_kv_at", "x100_gguf_get_int", "x100_gguf_get_float", "x100_gguf_get_str",
    "x100_gguf_get_arr_str", "x100_gguf_qwen3moe_params", "x100_gguf_type_name", "x100_gguf_block_bytes",
    "x100_gguf_block_elems", "x100_gguf_upload", "x100_gguf_pack_rows",
    "x100_attn_decode_hip", "x100_decode_layer_hip", "x100_decode_workspace_bytes",
    "x100_attn_decode_hip_ws", "x100_decode_layer_hip_ws",
)

GEMM_AUTO, GEMM_TILE256, GEMM_TILE128, GEMM_SKINNY, GEMM_GENERIC, GEMM_TILE256_W4, GEMM_TILE64, GEMM_TILE32 = \
    0, 1, 2, 3, 4, 5, 6, 7
GEMM_SET = 16   # variant flag: the overwrite form C = A*B (X100_GEMM_SET)


class X100Error(RuntimeError):
    def __init__(self, fn, code, text):
        super().__init__("%s failed: %d (%s)" % (fn, code, text))
        self.code = code


class Caps(ctypes.Structure):
    _fields_ = [
        ("device", ctypes.c_int), ("name", ctypes.c_char * 256), ("arch", ctypes.c_char * 64),
        ("cu_count", ctypes.c_int), ("clock_khz", ctypes.c_int), ("hbm_bytes", ctypes.c_size_t),
        ("lds_bytes", ctypes.c_int), ("l2_bytes", ctypes.c_int), ("is_gfx950", ctypes.c_int),
    ]


class LayerCfg(ctypes.Structure):
    """x100_layer_cfg (x100_decode.h)."""
    _fields_ = [(n, ctypes.c_int) for n in ("d", "n_head", "n_head_kv", "head_dim", "ff", "n_exp", "n_act", "ctx")] + \
               [("eps", ctypes.c_float), ("rope_base", ctypes.c_float)] + \
               [(n, ctypes.c_int) for n in ("wq_type", "wk_type", "wv_type", "wo_type")]


class LayerWeights(ctypes.Structure):
    """x100_layer_weights (x100_decode.h): device pointers."""
    _fields_ = [(n, ctypes.c_void_p) for n in ("attn_norm", "q_norm", "k_norm", "ffn_norm", "wq", "wk", "wv", "wo",
                                               "router", "wg", "wu", "wd", "k_cache", "v_cache")]


_lib = None


def lib():
    """Load libx100hip.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise FileNotFoundError("libx100hip.so not built: run __graft_entry__.build() "
                                "(make -C x100-gemm_amd)")
    L = ctypes.CDLL(LIB_PATH)
    i, p, sz = ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t
    L.gemm_ime_i8.argtypes = [i, i, i, p, p, p]
    L.gemm_ime_i8.restype = None
    L.gemm_hip_i8.argtypes = [i, i, i, p, p, p]
    L.gemm_hip_i8_dev.argtypes = [i, i, i, p, p, p, p]
    L.gemm_hip_i8_dev_variant.argtypes = [i, i, i, p, p, p, p, i]
    L.gemm_hip_i8_dev_set.argtypes = [i, i, i, p, p, p, p]
    L.x100_hip_detect.argtypes = [ctypes.POINTER(Caps)]
    L.x100_hip_caps_print.argtypes = [ctypes.POINTER(Caps)]
    L.x100_hip_caps_print.restype = None
    L.x100_hip_strerror.argtypes = [i]
    L.x100_hip_strerror.restype = ctypes.c_char_p
    L.x100q_gguf_bytes.argtypes = [i, i, i]
    L.x100q_gguf_bytes.restype = sz
    L.x100q_packed_bytes.argtypes = [i, i, i]
    L.x100q_packed_bytes.restype = sz
    L.x100q_pack.argtypes = [i, i, i, p, p, p]
    L.qgemv_hip.argtypes = [i, i, i, i, p, p, p, p]
    L.x100q_check_quant_div.argtypes = [ctypes.c_uint32, ctypes.c_uint32, p, p]
    L.moe_layer_hip.argtypes = [i, i, i, i, i, p, p, p, p, p, p, i, p, p, p]
    L.moe_layer_workspace_bytes.argtypes = [i, i, i, i, i]
    L.moe_layer_workspace_bytes.restype = sz
    L.moe_layer_hip_ws.argtypes = [i, i, i, i, i, p, p, p, p, p, p, i, p, p, p, sz, p]
    L.moe_layer_hip_noalloc.argtypes = [i, i, i, i, i, p, p, p, p, p, p, i, p, p, p]
    L.moe_pack_experts.argtypes = [i, i, i, p, p, p]
    L.x100_tile_bytes.argtypes = [i, i, i]
    L.x100_tile_bytes.restype = sz
    L.x100_pack_w_int4.argtypes = [i, i, p, p]
    L.x100_pack_w_int8.argtypes = [i, i, p, p]
    L.gemv_int4_hip.argtypes = [i, i, i, p, p, p, p]
    L.gemv_int8_hip.argtypes = [i, i, i, p, p, p, p]
    # GGUF reader (x100_gguf.h); the structures are declared in gguf.py
    u32, u64, i64, cp = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int64, ctypes.c_char_p
    L.x100_gguf_open.argtypes = [cp, ctypes.POINTER(p)]
    L.x100_gguf_close.argtypes = [p]
    L.x100_gguf_close.restype = None
    for name, rt in (("x100_gguf_version", u32), ("x100_gguf_n_tensors", i64), ("x100_gguf_n_kv", i64),
                     ("x100_gguf_alignment", u32), ("x100_gguf_data_offset", u64)):
        getattr(L, name).argtypes = [p]
        getattr(L, name).restype = rt
    L.x100_gguf_tensor_at.argtypes = [p, i64, p]
    L.x100_gguf_find.argtypes = [p, cp, p]
    L.x100_gguf_kv_at.argtypes = [p, i64, ctypes.POINTER(cp), ctypes.POINTER(u32), ctypes.POINTER(u32),
                                  ctypes.POINTER(u64)]
    L.x100_gguf_get_int.argtypes = [p, cp, ctypes.POINTER(i64)]
    L.x100_gguf_get_float.argtypes = [p, cp, ctypes.POINTER(ctypes.c_double)]
    L.x100_gguf_get_str.argtypes = [p, cp, ctypes.POINTER(p), ctypes.POINTER(u64)]
    L.x100_gguf_get_arr_str.argtypes = [p, cp, u64, ctypes.POINTER(p), ctypes.POINTER(u64)]
    L.x100_gguf_qwen3moe_params.argtypes = [p, p]
    L.x100_gguf_type_name.argtypes = [u32]
    L.x100_gguf_type_name.restype = cp
    L.x100_gguf_block_bytes.argtypes = [u32]
    L.x100_gguf_block_bytes.restype = sz
    L.x100_gguf_block_elems.argtypes = [u32]
    L.x100_gguf_upload.argtypes = [p, p, u64, u64, p, p]
    L.x100_gguf_pack_rows.argtypes = [p, p, u64, u64, p, p]
    for name in ("x100_gguf_open", "x100_gguf_tensor_at", "x100_gguf_find", "x100_gguf_kv_at",
                 "x100_gguf_get_int", "x100_gguf_get_float", "x100_gguf_get_str", "x100_gguf_get_arr_str",
                 "x100_gguf_qwen3moe_params", "x100_gguf_block_elems", "x100_gguf_upload",
                 "x100_gguf_pack_rows"):
        getattr(L, name).restype = i
    L.x100_attn_decode_hip.argtypes = [ctypes.POINTER(LayerCfg), ctypes.POINTER(LayerWeights), i, p, p]
    L.x100_decode_layer_hip.argtypes = [ctypes.POINTER(LayerCfg), ctypes.POINTER(LayerWeights), i, p, p, p, p]
    L.x100_attn_decode_hip.restype = i
    L.x100_decode_layer_hip.restype = i
    L.x100_decode_workspace_bytes.argtypes = [ctypes.POINTER(LayerCfg)]
    L.x100_decode_workspace_bytes.restype = sz
    L.x100_attn_decode_hip_ws.argtypes = [ctypes.POINTER(LayerCfg), ctypes.POINTER(LayerWeights), i, p, p, sz, p]
    L.x100_decode_layer_hip_ws.argtypes = [ctypes.POINTER(LayerCfg), ctypes.POINTER(LayerWeights), i, p, p, p, p, sz,
                                           p]
    L.x100_attn_decode_hip_ws.restype = i
    L.x100_decode_layer_hip_ws.restype = i
    for name in ("gemm_hip_i8", "gemm_hip_i8_dev", "gemm_hip_i8_dev_set", "gemm_hip_i8_dev_variant", "x100_hip_detect",
                 "x100q_pack", "qgemv_hip", "x100q_check_quant_div", "moe_layer_hip", "moe_layer_hip_ws", "moe_layer_hip_noalloc",
                 "moe_pack_experts",
                 "x100_pack_w_int4",
                 "x100_pack_w_int8",
                 "gemv_int4_hip", "gemv_int8_hip"):
        getattr(L, name).restype = i
    _lib = L
    return L


def _check(fn, rc):
    if rc != X100_OK:
        raise X100Error(fn, rc, lib().x100_hip_strerror(rc).decode())
    return rc


def strerror(code):
    return lib().x100_hip_strerror(code).decode()


def caps():
    c = Caps()
    _check("x100_hip_detect", lib().x100_hip_detect(ctypes.byref(c)))
    return c


# ---- int8 GEMM ---------------------------------------------------------------------------------
def gemm_dev(M, N, K, dA, dB, dC, stream=None, variant=GEMM_AUTO):
    """C += A*B on device pointers (ints); asynchronous on stream."""
    return _check("gemm_hip_i8_dev_variant",
                  lib().gemm_hip_i8_dev_variant(M, N, K, dA, dB, dC, stream, variant))


def gemm_dev_set(M, N, K, dA, dB, dC, stream=None, variant=None):
    """C = A*B (overwrite form) on device pointers; asynchronous on stream.  With a variant, that
    kernel choice through gemm_hip_i8_dev_variant(variant | GEMM_SET)."""
    if variant is None:
        return _check("gemm_hip_i8_dev_set", lib().gemm_hip_i8_dev_set(M, N, K, dA, dB, dC, stream))
    return _check("gemm_hip_i8_dev_variant",
                  lib().gemm_hip_i8_dev_variant(M, N, K, dA, dB, dC, stream, variant | GEMM_SET))


def gemm_host(A, B, C):
    """Drop-in host path: C (int32, MxN) += A (int8, MxK) . B (int8, KxN), numpy arrays."""
    M, K = A.shape
    K2, N = B.shape
    assert K == K2 and C.shape == (M, N)
    A = np.ascontiguousarray(A, dtype=np.int8)
    B = np.ascontiguousarray(B, dtype=np.int8)
    assert C.dtype == np.int32 and C.flags.c_contiguous
    return _check("gemm_hip_i8", lib().gemm_hip_i8(M, N, K, A.ctypes.data, B.ctypes.data,
                                                   C.ctypes.data))


# ---- quantized GEMV ----------------------------------------------------------------------------
def gguf_bytes(qtype, N, K):
    return lib().x100q_gguf_bytes(qtype, N, K)


def packed_bytes(qtype, N, K):
    return lib().x100q_packed_bytes(qtype, N, K)


def pack(qtype, N, K, d_src, d_dst, stream=None):
    return _check("x100q_pack", lib().x100q_pack(qtype, N, K, d_src, d_dst, stream))


def qgemv(qtype, M, N, K, d_w, d_x, d_y, stream=None):
    return _check("qgemv_hip", lib().qgemv_hip(qtype, M, N, K, d_w, d_x, d_y, stream))


def check_quant_div(lo_bits, hi_bits, d_counts, stream=None):
    return _check("x100q_check_quant_div", lib().x100q_check_quant_div(lo_bits, hi_bits, d_counts, stream))


# ---- MoE layer ---------------------------------------------------------------------------------
MOE_RESIDUAL, MOE_TILED = 1, 2


def _moe_flags(residual, tiled):
    return (MOE_RESIDUAL if residual else 0) | (MOE_TILED if tiled else 0)


def moe_pack_experts(n_exp, rows, K, d_src, d_dst, stream=None):
    """Q4_K expert tensor (n_exp x rows x K, ggml layout) -> the tiled layout (same size)."""
    return _check("moe_pack_experts", lib().moe_pack_experts(n_exp, rows, K, d_src, d_dst, stream))


def moe_layer(M, d, ff, n_exp, n_act, d_hn, d_R, d_Wg, d_Wu, d_Wd, d_out, residual=False,
              d_sel=None, d_sw=None, stream=None, tiled=False):
    return _check("moe_layer_hip",
                  lib().moe_layer_hip(M, d, ff, n_exp, n_act, d_hn, d_R, d_Wg, d_Wu, d_Wd, d_out,
                                      _moe_flags(residual, tiled), d_sel, d_sw, stream))


def moe_layer_noalloc(M, d, ff, n_exp, n_act, d_hn, d_R, d_Wg, d_Wu, d_Wd, d_out, residual=False,
                      d_sel=None, d_sw=None, stream=None, tiled=False):
    """moe_layer with the library's static per-GPU scratch (allocates nothing)."""
    return _check("moe_layer_hip_noalloc",
                  lib().moe_layer_hip_noalloc(M, d, ff, n_exp, n_act, d_hn, d_R, d_Wg, d_Wu, d_Wd, d_out,
                                              _moe_flags(residual, tiled), d_sel, d_sw, stream))


def moe_workspace_bytes(M, d, ff, n_exp, n_act):
    return lib().moe_layer_workspace_bytes(M, d, ff, n_exp, n_act)


def moe_layer_ws(M, d, ff, n_exp, n_act, d_hn, d_R, d_Wg, d_Wu, d_Wd, d_out, residual, d_sel, d_sw, d_ws, ws_bytes,
                 stream=None, tiled=False):
    """moe_layer on caller scratch (d_ws: device buffer of ws_bytes >= moe_workspace_bytes)."""
    return _check("moe_layer_hip_ws",
                  lib().moe_layer_hip_ws(M, d, ff, n_exp, n_act, d_hn, d_R, d_Wg, d_Wu, d_Wd, d_out,
                                         _moe_flags(residual, tiled), d_sel, d_sw, d_ws, ws_bytes, stream))


# ---- integer tile GEMV (int4 / int8 weights) ---------------------------------------------------
def tile_bytes(int4, N, K):
    return lib().x100_tile_bytes(1 if int4 else 0, N, K)


def pack_w(int4, W):
    """Host packer with the reference's tile layout (pack_w_int4 / pack_w_int8); W int8 N x K."""
    W = np.ascontiguousarray(W, dtype=np.int8)
    N, K = W.shape
    out = np.zeros(tile_bytes(int4, N, K), np.uint8 if int4 else np.int8)
    if int4:
        _check("x100_pack_w_int4", lib().x100_pack_w_int4(N, K, W.ctypes.data, out.ctypes.data))
    else:
        _check("x100_pack_w_int8", lib().x100_pack_w_int8(N, K, W.ctypes.data, out.ctypes.data))
    return out


def gemv_tile(int4, M, N, K, d_w, d_x, d_y, stream=None):
    """y[M][N] (int32) = W . x^T on device pointers; W packed by pack_w."""
    if int4:
        return _check("gemv_int4_hip", lib().gemv_int4_hip(M, N, K, d_w, d_x, d_y, stream))
    return _check("gemv_int8_hip", lib().gemv_int8_hip(M, N, K, d_w, d_x, d_y, stream))


# ---- decode layer (x100_decode.h) -----------------------------------------------------------------
def attn_decode(cfg, weights, pos, d_h, stream=None):
    """h += Wo.attention(...) for one token at pos; k, v written into the caches."""
    return _check("x100_attn_decode_hip", lib().x100_attn_decode_hip(ctypes.byref(cfg), ctypes.byref(weights), pos,
                                                                     d_h, stream))


def decode_layer(cfg, weights, pos, d_h, d_sel=None, d_sw=None, stream=None):
    """One whole decoder layer (attention half, then h += MoE(rmsnorm(h)))."""
    return _check("x100_decode_layer_hip", lib().x100_decode_layer_hip(ctypes.byref(cfg), ctypes.byref(weights), pos,
                                                                       d_h, d_sel, d_sw, stream))


def decode_workspace_bytes(cfg):
    return lib().x100_decode_workspace_bytes(ctypes.byref(cfg))


def attn_decode_ws(cfg, weights, pos, d_h, d_ws, ws_bytes, stream=None):
    return _check("x100_attn_decode_hip_ws", lib().x100_attn_decode_hip_ws(ctypes.byref(cfg), ctypes.byref(weights),
                                                                           pos, d_h, d_ws, ws_bytes, stream))


def decode_layer_ws(cfg, weights, pos, d_h, d_sel, d_sw, d_ws, ws_bytes, stream=None):
    return _check("x100_decode_layer_hip_ws", lib().x100_decode_layer_hip_ws(ctypes.byref(cfg), ctypes.byref(weights),
                                                                             pos, d_h, d_sel, d_sw, d_ws, ws_bytes,
                                                                             stream))
