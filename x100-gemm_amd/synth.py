"""Deterministic synthetic inputs for the quantized matrix-product path.

One generator family for every workload: splitmix64 for uniform bits, Box-Muller for N(0,1).
The same seeds give the same bytes in tests, bench.py and smoke().  Block layouts are the
GGUF-native ones (Q4_0 18 B / 32, Q8_0 34 B / 32, Q4_K 144 B / 256, Q3_K 110 B / 256,
Q5_K 176 B / 256, Q6_K 210 B / 256).

Workloads (sizes as named by the reference's measured shapes):
  int8 GEMM    A (MxK), B (KxN) i.i.d. uniform int8 in [-128, 127]
  Q4_0 weight  per 32-block: fp16 d = |N(0,1)|*0.01, 16 random bytes of nibbles
  Q4_K weight  per 256-block: fp16 d, dmin = |N(0,1)|*0.01, 12 random scale bytes, 128 nibble bytes
  Q3_K weight  per 256-block: 32 hmask + 64 qs + 12 scale random bytes, fp16 d = |N(0,1)|*0.01
  Q8_0 weight  per 32-block: fp16 d = |N(0,1)|*0.01, 32 random int8
  Q5_K weight  per 256-block: fp16 d, dmin = |N(0,1)|*0.001, 12 scale + 32 qh + 128 qs random bytes
  Q6_K weight  per 256-block: 128 ql + 64 qh random bytes, 16 random int8 scales,
               fp16 d = |N(0,1)|*0.0002
  (the Q5_K / Q6_K step sizes keep element magnitudes near those of the other formats, about
  0.1, as random 6-bit values times random 8-bit scales would otherwise reach 100)
  activations  fp32 N(0,1);  MoE router fp32 N(0, 0.02)
"""
import numpy as np

_GOLD = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)

Q4_0, Q8_0, Q3_K, Q4_K, Q5_K, Q6_K = 2, 8, 11, 12, 13, 14
BLOCK_BYTES = {Q4_0: 18, Q8_0: 34, Q4_K: 144, Q3_K: 110, Q5_K: 176, Q6_K: 210}
BLOCK_ELEMS = {Q4_0: 32, Q8_0: 32, Q4_K: 256, Q3_K: 256, Q5_K: 256, Q6_K: 256}

DT_Q4_0 = np.dtype([("d", "<u2"), ("qs", "u1", (16,))])
DT_Q4_K = np.dtype([("d", "<u2"), ("dmin", "<u2"), ("scales", "u1", (12,)), ("qs", "u1", (128,))])
DT_Q3_K = np.dtype([("hmask", "u1", (32,)), ("qs", "u1", (64,)), ("scales", "u1", (12,)), ("d", "<u2")])
DT_Q8_0 = np.dtype([("d", "<u2"), ("qs", "i1", (32,))])
DT_Q5_K = np.dtype([("d", "<u2"), ("dmin", "<u2"), ("scales", "u1", (12,)), ("qh", "u1", (32,)),
                    ("qs", "u1", (128,))])
DT_Q6_K = np.dtype([("ql", "u1", (128,)), ("qh", "u1", (64,)), ("scales", "i1", (16,)), ("d", "<u2")])
assert DT_Q4_0.itemsize == 18 and DT_Q4_K.itemsize == 144 and DT_Q3_K.itemsize == 110
assert DT_Q8_0.itemsize == 34 and DT_Q5_K.itemsize == 176 and DT_Q6_K.itemsize == 210


def splitmix64(seed, n):
    """n consecutive splitmix64 outputs for a 64-bit seed (uint64 array)."""
    with np.errstate(over="ignore"):
        i = np.arange(1, n + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + i * _GOLD
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def rand_bytes(seed, n):
    """n uniform random bytes (uint8)."""
    words = splitmix64(seed, (n + 7) // 8)
    return words.view(np.uint8)[:n].copy()


def rand_int8(seed, shape):
    n = int(np.prod(shape))
    return rand_bytes(seed, n).view(np.int8).reshape(shape)


def rand_normal(seed, n):
    """n standard normals (float64) by Box-Muller on 53-bit uniforms."""
    m = (n + 1) // 2
    z = splitmix64(seed, 2 * m)
    u1 = (z[0::2] >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    u2 = (z[1::2] >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    r = np.sqrt(-2.0 * np.log1p(-u1))
    t = 2.0 * np.pi * u2
    out = np.empty(2 * m, dtype=np.float64)
    out[0::2] = r * np.cos(t)
    out[1::2] = r * np.sin(t)
    return out[:n]


def normal_f32(seed, shape, std=1.0):
    n = int(np.prod(shape))
    return (rand_normal(seed, n) * std).astype(np.float32).reshape(shape)


def _scale_f16(seed, n, mult=0.01):
    return (np.abs(rand_normal(seed, n)) * mult).astype(np.float32).astype(np.float16).view(np.uint16)


def gemm_inputs(M, N, K, seed=2026):
    """A (MxK) and B (KxN) int8 uniform in [-128, 127]."""
    return rand_int8(seed, (M, K)), rand_int8(seed + 1, (K, N))


def quant_weight(qtype, N, K, seed):
    """N x K weight matrix as GGUF-native blocks: structured array of shape (N, K // QK)."""
    qk = BLOCK_ELEMS[qtype]
    if K % qk:
        raise ValueError("K must be a multiple of %d" % qk)
    nb = N * (K // qk)
    if qtype == Q4_0:
        w = np.zeros(nb, dtype=DT_Q4_0)
        w["d"] = _scale_f16(seed, nb)
        w["qs"] = rand_bytes(seed + 1, nb * 16).reshape(nb, 16)
    elif qtype == Q4_K:
        w = np.zeros(nb, dtype=DT_Q4_K)
        w["d"] = _scale_f16(seed, nb)
        w["dmin"] = _scale_f16(seed + 1, nb)
        w["scales"] = rand_bytes(seed + 2, nb * 12).reshape(nb, 12)
        w["qs"] = rand_bytes(seed + 3, nb * 128).reshape(nb, 128)
    elif qtype == Q3_K:
        w = np.zeros(nb, dtype=DT_Q3_K)
        w["hmask"] = rand_bytes(seed + 2, nb * 32).reshape(nb, 32)
        w["qs"] = rand_bytes(seed + 3, nb * 64).reshape(nb, 64)
        w["scales"] = rand_bytes(seed + 4, nb * 12).reshape(nb, 12)
        w["d"] = _scale_f16(seed, nb)
    elif qtype == Q8_0:
        w = np.zeros(nb, dtype=DT_Q8_0)
        w["d"] = _scale_f16(seed, nb)
        w["qs"] = rand_bytes(seed + 1, nb * 32).view(np.int8).reshape(nb, 32)
    elif qtype == Q5_K:
        w = np.zeros(nb, dtype=DT_Q5_K)
        w["d"] = _scale_f16(seed, nb, 0.001)
        w["dmin"] = _scale_f16(seed + 1, nb, 0.001)
        w["scales"] = rand_bytes(seed + 2, nb * 12).reshape(nb, 12)
        w["qh"] = rand_bytes(seed + 3, nb * 32).reshape(nb, 32)
        w["qs"] = rand_bytes(seed + 4, nb * 128).reshape(nb, 128)
    elif qtype == Q6_K:
        w = np.zeros(nb, dtype=DT_Q6_K)
        w["ql"] = rand_bytes(seed + 2, nb * 128).reshape(nb, 128)
        w["qh"] = rand_bytes(seed + 3, nb * 64).reshape(nb, 64)
        w["scales"] = rand_bytes(seed + 4, nb * 16).view(np.int8).reshape(nb, 16)
        w["d"] = _scale_f16(seed, nb, 0.0002)
    else:
        raise ValueError("unsupported qtype %r" % qtype)
    return w.reshape(N, K // qk)


def moe_weights(n_exp, d, ff, seed):
    """Expert tensors in the ggml 3-D layout (experts outermost), Q4_K:
    gate, up: (n_exp, ff, d/256) blocks; down: (n_exp, d, ff/256) blocks."""
    wg = quant_weight(Q4_K, n_exp * ff, d, seed).reshape(n_exp, ff, d // 256)
    wu = quant_weight(Q4_K, n_exp * ff, d, seed + 100).reshape(n_exp, ff, d // 256)
    wd = quant_weight(Q4_K, n_exp * d, ff, seed + 200).reshape(n_exp, d, ff // 256)
    return wg, wu, wd


def moe_router(n_exp, d, seed):
    return normal_f32(seed, (n_exp, d), std=0.02)


def decode_layer_weights(d, n_head, n_head_kv, head_dim, ff, n_exp, types, seed):
    """One Qwen3-MoE decoder layer: norms (fp32, around 1), attention weights in the given ggml
    types (types = (q, k, v, o); Wq n_head*head_dim x d, Wk / Wv n_head_kv*head_dim x d, Wo
    d x n_head*head_dim, GGUF blocks), router fp32 N(0, 0.02) [n_exp][d], Q4_K experts."""
    qd, kvd = n_head * head_dim, n_head_kv * head_dim
    L = {
        "attn_norm": (1.0 + 0.1 * normal_f32(seed, (d,))).astype(np.float32),
        "q_norm": (1.0 + 0.1 * normal_f32(seed + 1, (head_dim,))).astype(np.float32),
        "k_norm": (1.0 + 0.1 * normal_f32(seed + 2, (head_dim,))).astype(np.float32),
        "ffn_norm": (1.0 + 0.1 * normal_f32(seed + 3, (d,))).astype(np.float32),
        "wq": quant_weight(types[0], qd, d, seed + 10),
        "wk": quant_weight(types[1], kvd, d, seed + 20),
        "wv": quant_weight(types[2], kvd, d, seed + 30),
        "wo": quant_weight(types[3], d, qd, seed + 40),
        "router": moe_router(n_exp, d, seed + 50),
    }
    L["wg"], L["wu"], L["wd"] = moe_weights(n_exp, d, ff, seed + 60)
    return L

