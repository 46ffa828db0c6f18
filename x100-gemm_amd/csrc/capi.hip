// C-ABI of libx100hip: argument checking, device state and the host-pointer convenience paths.
// The kernels live in gemm_i8.hip, gemv_tile.hip, qgemv.hip and moe.hip.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <condition_variable>
#include <mutex>
#include <thread>
#include <vector>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

// Only the extern "C" entry points are exported (the library is built with -fvisibility=hidden).
#pragma GCC visibility push(default)
#include "x100_decode.h"
#include "x100_gemm.h"
#include "x100_gemv_tile.h"
#include "x100_gguf.h"
#include "x100_moe.h"
#include "x100_qgemv.h"
#pragma GCC visibility pop
#include "x100_internal.h"

namespace {

thread_local hipError_t g_last_hip = hipSuccess;

int hip_fail(hipError_t e)
{
    g_last_hip = e;
    if (e == hipErrorOutOfMemory) return X100_ENOMEM;
    if (e == hipErrorNoDevice || e == hipErrorInvalidDevice) return X100_ENODEV;
    return X100_EHIP;
}

#define X100_TRY(expr)                                                                             \
    do {                                                                                           \
        hipError_t e_ = (expr);                                                                    \
        if (e_ != hipSuccess) return hip_fail(e_);                                                 \
    } while (0)

// Every entry point checks once per thread that the current device is a gfx950 part: the kernels
// are built for gfx950 only, and there is no CPU fallback.
int check_device()
{
    thread_local int checked_dev = -1;
    int dev = 0;
    X100_TRY(hipGetDevice(&dev));
    if (dev == checked_dev) return X100_OK;
    hipDeviceProp_t p;
    X100_TRY(hipGetDeviceProperties(&p, dev));
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0) {
        g_last_hip = hipErrorInvalidDeviceFunction;
        return X100_ENODEV;
    }
    checked_dev = dev;
    return X100_OK;
}

// Workspaces of the convenience entry points (moe_layer_hip, x100_attn_decode_hip,
// x100_decode_layer_hip), one per (device, stream), so that calls on different streams never
// share scratch.  hipStreamPerThread is one handle for a distinct stream in every host thread, so
// for it the calling thread is part of the key as well.  A workspace only grows: the larger one
// is allocated with hipMalloc and the old one is kept until the process ends (never freed, no
// synchronisation), because work already queued on the stream, or a graph captured earlier at a
// smaller shape, may still use it.  Workspaces are not released when their stream is destroyed
// either (the library cannot see that); each is at most a few MB at decode shapes.  The kernels
// write every workspace byte they read within the same call, so the contents never need clearing.
// Growth is impossible while the stream is being captured: such a call returns X100_EINVAL
// (callers that capture graphs use the _ws entry points with their own scratch).
struct StreamWs {
    int dev;
    hipStream_t stream;
    std::thread::id thread;   // the calling thread for hipStreamPerThread, else a default id
    void *ptr;
    size_t bytes;
};
std::mutex g_ws_mu;
std::vector<StreamWs> g_ws;       // live workspace per (device, stream)
std::vector<void *> g_ws_retired;  // outgrown workspaces, kept alive

int stream_workspace(hipStream_t stream, size_t need, void **out)
{
    int dev = 0;
    X100_TRY(hipGetDevice(&dev));
    const std::thread::id tid = stream == hipStreamPerThread ? std::this_thread::get_id() : std::thread::id();
    std::lock_guard<std::mutex> lk(g_ws_mu);
    StreamWs *w = nullptr;
    for (StreamWs &e : g_ws)
        if (e.dev == dev && e.stream == stream && e.thread == tid) w = &e;
    if (w && w->bytes >= need) {
        *out = w->ptr;
        return X100_OK;
    }
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (stream) X100_TRY(hipStreamIsCapturing(stream, &cs));
    if (cs != hipStreamCaptureStatusNone) return X100_EINVAL;
    size_t bytes = (size_t)1 << 20;
    while (bytes < need) bytes <<= 1;
    void *p = nullptr;
    X100_TRY(hipMalloc(&p, bytes));
    if (w) {
        g_ws_retired.push_back(w->ptr);
        w->ptr = p;
        w->bytes = bytes;
    } else {
        g_ws.push_back(StreamWs{dev, stream, tid, p, bytes});
    }
    *out = p;
    return X100_OK;
}

inline size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }

// Scratch of moe_layer_hip_noalloc: a fixed array in the library's device image, one copy per GPU
// (each GPU the library runs on holds it until the process ends).  In host code `scratch` only
// names the symbol; its device address, which differs per GPU, comes from hipGetSymbolAddress
// with that GPU current, once, and only that address is ever handed to kernels.  Calls on one
// GPU share the array; nothing in it needs clearing (the kernels write every byte they read
// within a call).
static __device__ __align__(256) uint8_t scratch[X100_MOE_NOALLOC_MAX_BYTES];

std::mutex g_scratch_mu;
void *g_scratch_ptr[64];   // device address of `scratch` per device ordinal (null until set up)

int static_scratch(void **out)
{
    int dev = 0;
    X100_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) return X100_ENODEV;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        X100_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return X100_EHIP;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return X100_OK;
}

// Shape checks of the MoE block (moe_layer_hip's contract in x100_moe.h).
bool moe_shape_ok(int M, int d, int ff, int n_exp, int n_act)
{
    if (M < 1 || M > X100_MOE_MAX_ROWS || n_act < 1 || n_act > 8 || n_exp < n_act || n_exp > 256) return false;
    return d > 0 && ff > 0 && d % 256 == 0 && ff % 256 == 0 && d <= 4096 && ff <= 4096;
}

bool moe_ptrs_ok(const float *hn, const float *R, const void *Wg, const void *Wu, const void *Wd, const float *out)
{
    if (!hn || !R || !Wg || !Wu || !Wd || !out) return false;
    return !(((uintptr_t)hn | (uintptr_t)R | (uintptr_t)Wg | (uintptr_t)Wu | (uintptr_t)Wd) & 15);
}

// Host copies of the host-pointer GEMM: one range split in nt equal parts, copied by the caller and
// nt - 1 worker threads (a pageable <-> pinned copy runs at 29 GB/s on one core, 76-80 GB/s on 4-8).
// The workers start on the first use and live until the process ends (the pool is never destroyed,
// so no thread can be waiting on a destroyed condition variable at exit).
class CopyPool {
public:
    explicit CopyPool(int nt) : nt_(nt)
    {
        for (int i = 1; i < nt_; i++) std::thread([this, i] { worker(i); }).detach();
    }
    void copy(void *dst, const void *src, size_t n)
    {
        if (nt_ == 1 || n < ((size_t)1 << 20)) {
            memcpy(dst, src, n);
            return;
        }
        {
            std::lock_guard<std::mutex> lk(mu_);
            dst_ = (uint8_t *)dst;
            src_ = (const uint8_t *)src;
            n_ = n;
            pending_ = nt_ - 1;
            gen_++;
        }
        cv_job_.notify_all();
        part(0);
        std::unique_lock<std::mutex> lk(mu_);
        cv_done_.wait(lk, [this] { return pending_ == 0; });
    }

private:
    void part(int i)
    {
        // ceil(n / nt) rounded up to 64 bytes: the nt parts cover all n bytes
        const size_t per = ((n_ + nt_ - 1) / nt_ + 63) & ~(size_t)63, b = std::min(n_, per * i), e = std::min(n_, b + per);
        if (e > b) memcpy(dst_ + b, src_ + b, e - b);
    }
    void worker(int i)
    {
        uint64_t seen = 0;
        for (;;) {
            {
                std::unique_lock<std::mutex> lk(mu_);
                cv_job_.wait(lk, [&] { return gen_ != seen; });
                seen = gen_;
            }
            part(i);
            std::lock_guard<std::mutex> lk(mu_);
            if (--pending_ == 0) cv_done_.notify_one();
        }
    }
    const int nt_;
    std::mutex mu_;
    std::condition_variable cv_job_, cv_done_;
    uint64_t gen_ = 0;
    int pending_ = 0;
    uint8_t *dst_ = nullptr;
    const uint8_t *src_ = nullptr;
    size_t n_ = 0;
};

// Device buffers, stream and pinned staging of the host-pointer GEMM (gemm_hip_i8 / gemm_ime_i8),
// per device.  The device buffers only grow (hipMalloc of the larger size; the old one is freed,
// which is safe because every call has synchronised its stream before returning) and are kept for
// the life of the process, so a caller timing gemm_ime_i8 in a loop pays for the PCIe copies and
// the kernel only.  The copies go through two pinned slots of HG_CHUNK bytes (hipHostMalloc, once):
// the host copy of one chunk into (out of) a slot overlaps the DMA of the other slot, and pinned
// DMA runs at about 57 GB/s where a pageable copy runs at 29 (H2D) and 18 GB/s (D2H).
constexpr size_t HG_CHUNK = (size_t)8 << 20;
struct HostGemmState {
    std::mutex mu;
    hipStream_t stream = nullptr;
    void *ab = nullptr, *c = nullptr;
    size_t ab_bytes = 0, c_bytes = 0;
    void *pin[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    CopyPool *pool = nullptr;
};
HostGemmState g_host_gemm[64];

// Stream, events, pinned slots and copy pool of a device's host GEMM state, made on first use.
int host_gemm_setup(HostGemmState &h)
{
    if (!h.stream) X100_TRY(hipStreamCreateWithFlags(&h.stream, hipStreamNonBlocking));
    for (int i = 0; i < 2; i++) {
        if (!h.ev[i]) X100_TRY(hipEventCreateWithFlags(&h.ev[i], hipEventDisableTiming));
        if (!h.pin[i]) X100_TRY(hipHostMalloc(&h.pin[i], HG_CHUNK, hipHostMallocDefault));
    }
    if (!h.pool) {
        const unsigned hc = std::thread::hardware_concurrency();
        h.pool = new CopyPool((int)std::max(1u, std::min(4u, hc)));
    }
    return X100_OK;
}

int host_gemm_grow(HostGemmState &h, size_t ab, size_t c)
{
    if (h.ab_bytes < ab) {
        if (h.ab) X100_TRY(hipFree(h.ab));
        h.ab = nullptr;
        h.ab_bytes = 0;
        X100_TRY(hipMalloc(&h.ab, ab));
        h.ab_bytes = ab;
    }
    if (h.c_bytes < c) {
        if (h.c) X100_TRY(hipFree(h.c));
        h.c = nullptr;
        h.c_bytes = 0;
        X100_TRY(hipMalloc(&h.c, c));
        h.c_bytes = c;
    }
    return X100_OK;
}

int moe_run(int M, int d, int ff, int n_exp, int n_act, const float *hn, const float *R, const void *Wg,
            const void *Wu, const void *Wd, float *out, int residual, int *sel, float *sw, void *ws, void *stream)
{
    hipError_t e = x100_moe_launch(M, d, ff, n_exp, n_act, hn, R, Wg, Wu, Wd, out, residual, sel, sw, ws,
                                   (hipStream_t)stream);
    if (e == hipErrorInvalidValue) return X100_EINVAL;
    if (e != hipSuccess) return hip_fail(e);
    return X100_OK;
}

}  // namespace

extern "C" {

// ---------------------------------------------------------------------------------------------
// int8 GEMM
// ---------------------------------------------------------------------------------------------
int gemm_hip_i8_dev_variant(int M, int N, int K, const int8_t *dA, const int8_t *dB, int32_t *dC,
                            void *stream, int variant)
{
    const bool set = (variant & X100_GEMM_SET) != 0;
    variant &= ~X100_GEMM_SET;
    if (M < 0 || N < 0 || K < 0 || variant < 0 || variant > 7) return X100_EINVAL;
    if (M == 0 || N == 0) return X100_OK;   // no output elements
    if (!dC || (K > 0 && (!dA || !dB))) return X100_EINVAL;
    if (K == 0 && !set) return X100_OK;     // C += (empty product) leaves C unchanged
    // Any K: from K = 2^17 a dot product can leave the int32 range, and then C wraps modulo 2^32
    // exactly as the reference's int32 accumulation does (integer addition modulo 2^32 is
    // associative, so the kernels' summation order does not matter).
    int rc = check_device();
    if (rc) return rc;
    hipError_t e = K == 0 ? x100_zero_i32_launch(dC, (size_t)M * N, (hipStream_t)stream)   // C = 0
                          : x100_gemm_i8_launch(M, N, K, dA, dB, dC, (hipStream_t)stream, variant, !set);
    if (e == hipErrorInvalidValue) return X100_EINVAL;
    if (e != hipSuccess) return hip_fail(e);
    return X100_OK;
}

int gemm_hip_i8_dev(int M, int N, int K, const int8_t *dA, const int8_t *dB, int32_t *dC,
                    void *stream)
{
    return gemm_hip_i8_dev_variant(M, N, K, dA, dB, dC, stream, X100_GEMM_AUTO);
}

int gemm_hip_i8_dev_set(int M, int N, int K, const int8_t *dA, const int8_t *dB, int32_t *dC, void *stream)
{
    return gemm_hip_i8_dev_variant(M, N, K, dA, dB, dC, stream, X100_GEMM_AUTO | X100_GEMM_SET);
}

int gemm_hip_i8(int M, int N, int K, const int8_t *A, const int8_t *B, int32_t *C)
{
    if (M < 0 || N < 0 || K < 0) return X100_EINVAL;
    if (M == 0 || N == 0 || K == 0) return X100_OK;
    if (!A || !B || !C) return X100_EINVAL;
    int rc = check_device();
    if (rc) return rc;
    int dev = 0;
    X100_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) return X100_ENODEV;
    const size_t sa = (size_t)M * K, sb = (size_t)K * N, sc = (size_t)M * N * sizeof(int32_t);
    // One call at a time per device: the staging buffers and the stream are shared.
    HostGemmState &h = g_host_gemm[dev];
    std::lock_guard<std::mutex> lk(h.mu);
    rc = host_gemm_setup(h);
    if (rc) return rc;
    rc = host_gemm_grow(h, sa + sb, sc);
    if (rc) return rc;
    int8_t *dA = (int8_t *)h.ab, *dB = dA + sa;
    int32_t *dC = (int32_t *)h.c;
    // A, B, C in: chunk i is copied into slot i % 2 once that slot's previous DMA is done, then
    // DMA'd to the device.
    struct Piece {
        uint8_t *dev;
        const uint8_t *host;
        size_t bytes;
    };
    const Piece in[3] = {{(uint8_t *)dA, (const uint8_t *)A, sa}, {(uint8_t *)dB, (const uint8_t *)B, sb},
                         {(uint8_t *)dC, (const uint8_t *)C, sc}};
    int slot = 0;
    bool used[2] = {false, false};
    for (const Piece &pc : in)
        for (size_t off = 0; off < pc.bytes; off += HG_CHUNK) {
            const size_t len = std::min(HG_CHUNK, pc.bytes - off);
            if (used[slot]) X100_TRY(hipEventSynchronize(h.ev[slot]));
            h.pool->copy(h.pin[slot], pc.host + off, len);
            X100_TRY(hipMemcpyAsync(pc.dev + off, h.pin[slot], len, hipMemcpyHostToDevice, h.stream));
            X100_TRY(hipEventRecord(h.ev[slot], h.stream));
            used[slot] = true;
            slot ^= 1;
        }
    rc = gemm_hip_i8_dev(M, N, K, dA, dB, dC, h.stream);
    if (rc != X100_OK) {
        (void)hipStreamSynchronize(h.stream);
        return rc;
    }
    // C out: chunk i is DMA'd into slot i % 2 (after the kernel, in stream order) while the host
    // copies chunk i - 1 out of the other slot.
    const size_t nch = (sc + HG_CHUNK - 1) / HG_CHUNK;
    for (size_t i = 0; i <= nch; i++) {
        if (i < nch) {
            const size_t len = std::min(HG_CHUNK, sc - i * HG_CHUNK);
            X100_TRY(hipMemcpyAsync(h.pin[i & 1], (const uint8_t *)dC + i * HG_CHUNK, len, hipMemcpyDeviceToHost,
                                    h.stream));
            X100_TRY(hipEventRecord(h.ev[i & 1], h.stream));
        }
        if (i > 0) {
            const size_t j = i - 1, len = std::min(HG_CHUNK, sc - j * HG_CHUNK);
            X100_TRY(hipEventSynchronize(h.ev[j & 1]));
            h.pool->copy((uint8_t *)C + j * HG_CHUNK, h.pin[j & 1], len);
        }
    }
    X100_TRY(hipStreamSynchronize(h.stream));
    return X100_OK;
}

void gemm_ime_i8(int M, int N, int K, const int8_t *A, const int8_t *B, int32_t *C)
{
    int rc = gemm_hip_i8(M, N, K, A, B, C);
    if (rc != X100_OK) {
        fprintf(stderr, "gemm_ime_i8 (libx100hip): %s\n", x100_hip_strerror(rc));
        abort();
    }
}

// ---------------------------------------------------------------------------------------------
// caps / errors
// ---------------------------------------------------------------------------------------------
int x100_hip_detect(x100_hip_caps_t *caps)
{
    if (!caps) return X100_EINVAL;
    memset(caps, 0, sizeof(*caps));
    int n = 0;
    X100_TRY(hipGetDeviceCount(&n));
    if (n <= 0) return X100_ENODEV;
    int dev = 0;
    X100_TRY(hipGetDevice(&dev));
    hipDeviceProp_t p;
    X100_TRY(hipGetDeviceProperties(&p, dev));
    caps->device = dev;
    snprintf(caps->name, sizeof caps->name, "%s", p.name);
    snprintf(caps->arch, sizeof caps->arch, "%s", p.gcnArchName);
    caps->cu_count = p.multiProcessorCount;
    caps->clock_khz = p.clockRate;
    caps->hbm_bytes = p.totalGlobalMem;
    caps->lds_bytes = (int)p.sharedMemPerBlock;
    caps->l2_bytes = p.l2CacheSize;
    caps->is_gfx950 = strncmp(p.gcnArchName, "gfx950", 6) == 0;
    return X100_OK;
}

void x100_hip_caps_print(const x100_hip_caps_t *c)
{
    if (!c) return;
    printf("device %d: %s (%s)\n", c->device, c->name, c->arch);
    printf("  CUs %d  clock %.0f MHz  HBM %.1f GiB  LDS/block %d KiB  L2 %d KiB  gfx950 %s\n",
           c->cu_count, c->clock_khz / 1000.0, c->hbm_bytes / 1073741824.0, c->lds_bytes / 1024,
           c->l2_bytes / 1024, c->is_gfx950 ? "yes" : "no");
}

const char *x100_hip_strerror(int code)
{
    switch (code) {
    case X100_OK: return "ok";
    case X100_EINVAL: return "invalid argument or unsupported shape";
    case X100_ENODEV: return g_last_hip != hipSuccess ? hipGetErrorString(g_last_hip)
                                                      : "no gfx950 device";
    case X100_ENOMEM: return "device allocation failed";
    case X100_EHIP: return hipGetErrorString(g_last_hip);
    case X100_EIO: return "file could not be opened or mapped";
    case X100_EFORMAT: return "not a GGUF v2/v3 file, or a field lies outside the file";
    case X100_ENOTFOUND: return "no tensor or key of that name (or of that type)";
    case X100_ESCRATCH: return "the shape needs more scratch than the static array of moe_layer_hip_noalloc "
                               "holds (X100_MOE_NOALLOC_MAX_BYTES)";
    }
    return "unknown error";
}

// ---------------------------------------------------------------------------------------------
// quantized GEMV
// ---------------------------------------------------------------------------------------------
// Elements and bytes per GGUF block (bench/gguf_dump.c:12-13 type ids; block sizes of ggml).
static int qk_of(int qtype)
{
    switch (qtype) {
    case X100_Q4_0: case X100_Q8_0: return 32;
    case X100_Q3_K: case X100_Q4_K: case X100_Q5_K: case X100_Q6_K: return 256;
    }
    return 0;
}

static size_t block_bytes_of(int qtype)
{
    switch (qtype) {
    case X100_Q4_0: return 18;
    case X100_Q8_0: return 34;
    case X100_Q3_K: return 110;
    case X100_Q4_K: return 144;
    case X100_Q5_K: return 176;
    case X100_Q6_K: return 210;
    }
    return 0;
}

size_t x100q_gguf_bytes(int qtype, int N, int K)
{
    const int qk = qk_of(qtype);
    if (!qk || N < 0 || K <= 0 || K % qk) return 0;
    return (size_t)N * (K / qk) * block_bytes_of(qtype);
}

size_t x100q_packed_bytes(int qtype, int N, int K)
{
    if (!x100q_gguf_bytes(qtype, N, K)) return 0;
    return x100_q_packed_bytes(qtype, N, K);
}

int x100q_pack(int qtype, int N, int K, const void *w_gguf, void *w_packed, void *stream)
{
    if (!x100q_gguf_bytes(qtype, N, K) || !w_gguf || !w_packed || ((uintptr_t)w_packed & 255)) return X100_EINVAL;
    int rc = check_device();
    if (rc) return rc;
    hipError_t e = x100_q_pack_launch(qtype, N, K, w_gguf, w_packed, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e);
    return X100_OK;
}

int qgemv_hip(int qtype, int M, int N, int K, const void *w_packed, const float *x, float *y,
              void *stream)
{
    if (!x100q_gguf_bytes(qtype, N, K) || M < 1 || M > 8) return X100_EINVAL;
    if (N == 0) return X100_OK;
    if (!w_packed || !x || !y || ((uintptr_t)x & 15) || ((uintptr_t)w_packed & 255)) return X100_EINVAL;
    int rc = check_device();
    if (rc) return rc;
    hipError_t e = x100_qgemv_launch(qtype, M, N, K, w_packed, x, y, (hipStream_t)stream);
    if (e == hipErrorInvalidValue) return X100_EINVAL;
    if (e != hipSuccess) return hip_fail(e);
    return X100_OK;
}

int x100q_check_quant_div(uint32_t lo_bits, uint32_t hi_bits, unsigned long long *d_counts, void *stream)
{
    if (!d_counts || lo_bits > hi_bits || hi_bits > 0x7f7fffffu) return X100_EINVAL;
    int rc = check_device();
    if (rc) return rc;
    hipError_t e = x100_check_quant_div_launch(lo_bits, hi_bits, d_counts, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e);
    return X100_OK;
}

// ---------------------------------------------------------------------------------------------
// integer tile GEMV (int4 / int8 weights)
// ---------------------------------------------------------------------------------------------
size_t x100_tile_bytes(int int4, int N, int K)
{
    if (N <= 0 || K <= 0 || N % 8 || K % (int4 ? 32 : 16)) return 0;
    return int4 ? (size_t)N * K / 2 : (size_t)N * K;
}

int x100_pack_w_int4(int N, int K, const int8_t *W, uint8_t *Wq)
{
    if (!x100_tile_bytes(1, N, K) || !W || !Wq) return X100_EINVAL;
    const int kp_n = K / 32;
    for (int nb = 0; nb < N / 8; nb++)
        for (int kp = 0; kp < kp_n; kp++) {
            uint8_t *t = Wq + ((size_t)nb * kp_n + kp) * 128;
            for (int n = 0; n < 8; n++) {
                const int8_t *row = W + (size_t)(8 * nb + n) * K + 32 * kp;
                for (int k = 0; k < 16; k++)
                    t[16 * n + k] = (uint8_t)((row[k] & 0xf) | ((row[16 + k] & 0xf) << 4));
            }
        }
    return X100_OK;
}

int x100_pack_w_int8(int N, int K, const int8_t *W, int8_t *Wp)
{
    if (!x100_tile_bytes(0, N, K) || !W || !Wp) return X100_EINVAL;
    const int kb_n = K / 16;
    for (int nb = 0; nb < N / 8; nb++)
        for (int kb = 0; kb < kb_n; kb++) {
            int8_t *t = Wp + ((size_t)nb * kb_n + kb) * 128;
            for (int n = 0; n < 8; n++) memcpy(t + 16 * n, W + (size_t)(8 * nb + n) * K + 16 * kb, 16);
        }
    return X100_OK;
}

static int gemv_tile(int int4, int M, int N, int K, const void *W, const int8_t *x, int32_t *y, void *stream)
{
    if (!x100_tile_bytes(int4, N, K) || M < 1 || M > 8) return X100_EINVAL;
    if ((size_t)M * K + 16 + ((size_t)M * (K / 16) + 1) * 4 > 64 * 1024) return X100_EINVAL;
    if (!W || !x || !y || ((uintptr_t)W & 15) || ((uintptr_t)x & 15)) return X100_EINVAL;
    int rc = check_device();
    if (rc) return rc;
    hipError_t e = x100_gemv_tile_launch(int4, M, N, K, W, x, y, (hipStream_t)stream);
    if (e == hipErrorInvalidValue) return X100_EINVAL;
    if (e != hipSuccess) return hip_fail(e);
    return X100_OK;
}

int gemv_int4_hip(int M, int N, int K, const uint8_t *Wq, const int8_t *x, int32_t *y, void *stream)
{
    return gemv_tile(1, M, N, K, Wq, x, y, stream);
}

int gemv_int8_hip(int M, int N, int K, const int8_t *Wp, const int8_t *x, int32_t *y, void *stream)
{
    return gemv_tile(0, M, N, K, Wp, x, y, stream);
}

// ---------------------------------------------------------------------------------------------
// MoE decode layer
// ---------------------------------------------------------------------------------------------
size_t moe_layer_workspace_bytes(int M, int d, int ff, int n_exp, int n_act)
{
    if (!moe_shape_ok(M, d, ff, n_exp, n_act)) return 0;
    return al256(x100_moe_workspace_bytes(M, d, ff, n_exp, n_act));
}

int moe_layer_hip_ws(int M, int d, int ff, int n_exp, int n_act, const float *hn, const float *R, const void *Wg,
                     const void *Wu, const void *Wd, float *out, int residual, int *sel, float *sw, void *ws,
                     size_t ws_bytes, void *stream)
{
    if (!moe_shape_ok(M, d, ff, n_exp, n_act) || !moe_ptrs_ok(hn, R, Wg, Wu, Wd, out)) return X100_EINVAL;
    if (!ws || ((uintptr_t)ws & 255) || ws_bytes < moe_layer_workspace_bytes(M, d, ff, n_exp, n_act))
        return X100_EINVAL;
    int rc = check_device();
    if (rc) return rc;
    return moe_run(M, d, ff, n_exp, n_act, hn, R, Wg, Wu, Wd, out, residual, sel, sw, ws, stream);
}

int moe_layer_hip(int M, int d, int ff, int n_exp, int n_act, const float *hn, const float *R,
                  const void *Wg, const void *Wu, const void *Wd, float *out, int residual,
                  int *sel, float *sw, void *stream)
{
    if (!moe_shape_ok(M, d, ff, n_exp, n_act) || !moe_ptrs_ok(hn, R, Wg, Wu, Wd, out)) return X100_EINVAL;
    int rc = check_device();
    if (rc) return rc;
    const size_t need = moe_layer_workspace_bytes(M, d, ff, n_exp, n_act);
    void *ws = nullptr;
    rc = stream_workspace((hipStream_t)stream, need, &ws);
    if (rc) return rc;
    return moe_run(M, d, ff, n_exp, n_act, hn, R, Wg, Wu, Wd, out, residual, sel, sw, ws, stream);
}

int moe_pack_experts(int n_exp, int rows, int K, const void *src, void *dst, void *stream)
{
    if (n_exp < 1 || rows < 8 || rows % 8 || K < 256 || K % 256 || !src || !dst) return X100_EINVAL;
    if (((uintptr_t)src | (uintptr_t)dst) & 15) return X100_EINVAL;
    const size_t bytes = (size_t)n_exp * rows * (K / 256) * 144;
    const uintptr_t s0 = (uintptr_t)src, d0 = (uintptr_t)dst;
    if (s0 < d0 + bytes && d0 < s0 + bytes) return X100_EINVAL;   // the copy is not in place
    int rc = check_device();
    if (rc) return rc;
    hipError_t e = x100_moe_tile_pack(n_exp, rows, K, src, dst, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e);
    return X100_OK;
}

int moe_layer_hip_noalloc(int M, int d, int ff, int n_exp, int n_act, const float *hn, const float *R,
                          const void *Wg, const void *Wu, const void *Wd, float *out, int residual, int *sel,
                          float *sw, void *stream)
{
    if (!moe_shape_ok(M, d, ff, n_exp, n_act) || !moe_ptrs_ok(hn, R, Wg, Wu, Wd, out)) return X100_EINVAL;
    if (moe_layer_workspace_bytes(M, d, ff, n_exp, n_act) > X100_MOE_NOALLOC_MAX_BYTES) return X100_ESCRATCH;
    int rc = check_device();
    if (rc) return rc;
    void *ws = nullptr;
    if ((rc = static_scratch(&ws))) return rc;
    return moe_run(M, d, ff, n_exp, n_act, hn, R, Wg, Wu, Wd, out, residual, sel, sw, ws, stream);
}

// ---------------------------------------------------------------------------------------------
// decode layer
// ---------------------------------------------------------------------------------------------
// Every argument of the layer is checked here, before any kernel is enqueued, so that an error
// return leaves h and the caches untouched.
static int check_layer(const x100_layer_cfg *c, const x100_layer_weights *w, int pos, const float *h, bool moe)
{
    if (!c || !w || !h) return X100_EINVAL;
    if (c->d <= 0 || c->head_dim != 128 || c->n_head < 1 || c->n_head_kv < 1 || c->n_head % c->n_head_kv ||
        c->n_head / c->n_head_kv > 16 || c->ctx < 1 || pos < 0 || pos >= c->ctx || c->d > 65536 ||
        c->n_head > 1024)
        return X100_EINVAL;
    if ((size_t)c->n_head_kv * c->ctx * 128 >= ((size_t)1 << 40)) return X100_EINVAL;
    if (!w->attn_norm || !w->q_norm || !w->k_norm || !w->wq || !w->wk || !w->wv || !w->wo || !w->k_cache ||
        !w->v_cache)
        return X100_EINVAL;
    if (((uintptr_t)w->k_cache & 15) || ((uintptr_t)w->v_cache & 15)) return X100_EINVAL;
    const int qd = c->n_head * 128, kvd = c->n_head_kv * 128;
    if (!x100q_gguf_bytes(c->wq_type, qd, c->d) || !x100q_gguf_bytes(c->wk_type, kvd, c->d) ||
        !x100q_gguf_bytes(c->wv_type, kvd, c->d) || !x100q_gguf_bytes(c->wo_type, c->d, qd))
        return X100_EINVAL;
    if (!x100_qgemv_supported(c->wq_type, 1, qd, c->d) || !x100_qgemv_supported(c->wk_type, 1, kvd, c->d) ||
        !x100_qgemv_supported(c->wv_type, 1, kvd, c->d) || !x100_qgemv_supported(c->wo_type, 1, c->d, qd))
        return X100_EINVAL;
    if (((uintptr_t)w->wq | (uintptr_t)w->wk | (uintptr_t)w->wv | (uintptr_t)w->wo) & 255) return X100_EINVAL;
    if (moe) {
        if (!w->ffn_norm || !moe_shape_ok(1, c->d, c->ff, c->n_exp, c->n_act)) return X100_EINVAL;
        if (!w->router || !w->wg || !w->wu || !w->wd) return X100_EINVAL;
        if (((uintptr_t)w->router | (uintptr_t)w->wg | (uintptr_t)w->wu | (uintptr_t)w->wd) & 15) return X100_EINVAL;
    }
    return X100_OK;
}

static size_t attn_ws_bytes(const x100_layer_cfg *c) { return al256(x100_attn_workspace_bytes(c)); }

size_t x100_decode_workspace_bytes(const x100_layer_cfg *c)
{
    if (!c || c->d <= 0 || c->head_dim != 128 || c->n_head < 1 || c->n_head_kv < 1 || c->ctx < 1 || c->d > 65536 ||
        c->n_head > 1024)
        return 0;
    const size_t attn = attn_ws_bytes(c);
    // the MoE block's share when the configuration has one (the attention half alone needs less)
    return attn + moe_layer_workspace_bytes(1, c->d, c->ff, c->n_exp, c->n_act);
}

// The attention half on workspace ws; with w->ffn_norm set, *hn receives rmsnorm(h, ffn_norm).
static int attn_half(const x100_layer_cfg *c, const x100_layer_weights *w, int pos, float *h, float **hn, void *ws,
                     void *stream)
{
    hipError_t e = x100_attn_launch(c, w, pos, h, (float *)ws, hn, (hipStream_t)stream);
    if (e == hipErrorInvalidValue) return X100_EINVAL;
    if (e != hipSuccess) return hip_fail(e);
    return X100_OK;
}

static int attn_decode(const x100_layer_cfg *c, const x100_layer_weights *w, int pos, float *h, void *ws,
                       void *stream)
{
    x100_layer_weights w2 = *w;
    w2.ffn_norm = nullptr;   // the residual add only, no norm for a following block
    return attn_half(c, &w2, pos, h, nullptr, ws, stream);
}

// A layer: the attention half, then the MoE block on rmsnorm(h, ffn_norm) with the residual add.
// Where x100_moe_norm_launch takes the shape (d = 2048) and h and ffn_norm are 16-byte aligned (its
// router loads them as float4), h += o and the norm run inside its router kernel instead of a
// launch of their own (same bits).
static int decode_layer(const x100_layer_cfg *c, const x100_layer_weights *w, int pos, float *h, int *sel, float *sw,
                        void *ws, void *stream)
{
    void *mws = (uint8_t *)ws + attn_ws_bytes(c);
    if (w->ffn_norm && !(((uintptr_t)h | (uintptr_t)w->ffn_norm) & 15) &&
        x100_moe_norm_supported(c->d, c->ff, c->n_exp, c->n_act, X100_MOE_RESIDUAL)) {
        float *o = nullptr;
        hipError_t e = x100_attn_launch(c, w, pos, h, (float *)ws, nullptr, (hipStream_t)stream, &o);
        if (e == hipSuccess)
            e = x100_moe_norm_launch(c->d, c->ff, c->n_exp, c->n_act, h, o, w->ffn_norm, c->eps, w->router, w->wg,
                                     w->wu, w->wd, X100_MOE_RESIDUAL, sel, sw, mws, (hipStream_t)stream);
        if (e == hipErrorInvalidValue) return X100_EINVAL;
        if (e != hipSuccess) return hip_fail(e);
        return X100_OK;
    }
    float *hn = nullptr;
    int rc = attn_half(c, w, pos, h, &hn, ws, stream);
    if (rc) return rc;
    return moe_run(1, c->d, c->ff, c->n_exp, c->n_act, hn, w->router, w->wg, w->wu, w->wd, h, X100_MOE_RESIDUAL, sel,
                   sw, mws, stream);
}

int x100_attn_decode_hip_ws(const x100_layer_cfg *c, const x100_layer_weights *w, int pos, float *h, void *ws,
                            size_t ws_bytes, void *stream)
{
    int rc = check_layer(c, w, pos, h, false);
    if (rc) return rc;
    if (!ws || ((uintptr_t)ws & 255) || ws_bytes < attn_ws_bytes(c)) return X100_EINVAL;
    if ((rc = check_device())) return rc;
    return attn_decode(c, w, pos, h, ws, stream);
}

int x100_attn_decode_hip(const x100_layer_cfg *c, const x100_layer_weights *w, int pos, float *h, void *stream)
{
    int rc = check_layer(c, w, pos, h, false);
    if (rc) return rc;
    if ((rc = check_device())) return rc;
    void *ws = nullptr;
    if ((rc = stream_workspace((hipStream_t)stream, attn_ws_bytes(c), &ws))) return rc;
    return attn_decode(c, w, pos, h, ws, stream);
}

int x100_decode_layer_hip_ws(const x100_layer_cfg *c, const x100_layer_weights *w, int pos, float *h, int *sel,
                             float *sw, void *ws, size_t ws_bytes, void *stream)
{
    int rc = check_layer(c, w, pos, h, true);
    if (rc) return rc;
    if (!ws || ((uintptr_t)ws & 255) || ws_bytes < x100_decode_workspace_bytes(c)) return X100_EINVAL;
    if ((rc = check_device())) return rc;
    return decode_layer(c, w, pos, h, sel, sw, ws, stream);
}

int x100_decode_layer_hip(const x100_layer_cfg *c, const x100_layer_weights *w, int pos, float *h, int *sel,
                          float *sw, void *stream)
{
    int rc = check_layer(c, w, pos, h, true);
    if (rc) return rc;
    if ((rc = check_device())) return rc;
    void *ws = nullptr;
    if ((rc = stream_workspace((hipStream_t)stream, x100_decode_workspace_bytes(c), &ws))) return rc;
    return decode_layer(c, w, pos, h, sel, sw, ws, stream);
}

}  // extern "C"
