/*
 * x100_gguf.h -- GGUF v2/v3 checkpoint reader of libx100hip: maps a .gguf file read-only and hands
 * its block-quantized tensors to the GPU kernels in their native (GGUF) block order.
 *
 * Replaces the reference's loader `gguf_open` / `gguf_find` / `gguf_has` (qwen_moe.c:110-154,
 * the same code in qwen_moe_q3k.c:1084-1128) and the listing tool bench/gguf_dump.c.  Where the
 * reference dequantizes tensors to fp32 and re-encodes them into its vendor layouts
 * (gguf_dequant_into + the requant cache, qwen_moe.c:156-181, 233-269), these entry points upload
 * the GGUF bytes as they are: the GEMV and MoE kernels consume ggml blocks directly.
 *
 * Every read of the file is bounds-checked: a truncated or malformed file gives X100_EFORMAT,
 * never an access outside the mapping.  Handles are read-only after x100_gguf_open and may be
 * shared between threads.
 */
#ifndef X100_HIP_GGUF_H
#define X100_HIP_GGUF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define X100_EIO        -5   /* the file could not be opened or mapped                    */
#define X100_EFORMAT    -6   /* not a GGUF v2/v3 file, or a field lies outside the file   */
#define X100_ENOTFOUND  -7   /* no tensor / key of that name, or a key of another type    */

/* GGUF metadata value types (the u32 type field of a key/value pair). */
#define X100_GGUF_U8      0
#define X100_GGUF_I8      1
#define X100_GGUF_U16     2
#define X100_GGUF_I16     3
#define X100_GGUF_U32     4
#define X100_GGUF_I32     5
#define X100_GGUF_F32     6
#define X100_GGUF_BOOL    7
#define X100_GGUF_STRING  8
#define X100_GGUF_ARRAY   9
#define X100_GGUF_U64    10
#define X100_GGUF_I64    11
#define X100_GGUF_F64    12

typedef struct x100_gguf x100_gguf;          /* opaque handle */

typedef struct {
    const char *name;       /* NUL-terminated copy owned by the handle                        */
    uint32_t type;          /* ggml type id (bench/gguf_dump.c:12-14)                         */
    uint32_t n_dims;        /* 1..4                                                           */
    uint64_t dims[4];       /* ggml order: dims[0] is the contiguous (K) dimension            */
    uint64_t offset;        /* from the start of the tensor data section                      */
    uint64_t n_elems;       /* product of dims                                                */
    uint64_t n_bytes;       /* 0 for a type whose block size this library does not know       */
    const void *data;       /* host address inside the mapping, NULL when n_bytes is 0        */
} x100_gguf_tensor;

/* Model hyper-parameters read by the reference's gguf_open (qwen_moe.c:129-146), with its
 * defaults for absent keys: rope_base 1e6, n_exp 128, n_act 8, moe_ffn 768, others 0.  vocab is
 * dims[1] of token_embd.weight (qwen_moe.c:151). */
typedef struct {
    int block_count, embd, ffn, n_head, n_head_kv, head_dim, vocab, n_exp, n_act, moe_ffn;
    float rope_base;
    int n_tokens;           /* length of tokenizer.ggml.tokens, 0 if absent                   */
} x100_gguf_qwen3moe;

/* Open and parse; *out receives the handle (NULL on error). */
int x100_gguf_open(const char *path, x100_gguf **out);
void x100_gguf_close(x100_gguf *g);

uint32_t x100_gguf_version(const x100_gguf *g);
int64_t x100_gguf_n_tensors(const x100_gguf *g);
int64_t x100_gguf_n_kv(const x100_gguf *g);
uint32_t x100_gguf_alignment(const x100_gguf *g);      /* general.alignment, default 32 */
uint64_t x100_gguf_data_offset(const x100_gguf *g);    /* file offset of the tensor data */

/* Tensor i in file order, or by name (gguf_find / gguf_has, qwen_moe.c:153-154). */
int x100_gguf_tensor_at(const x100_gguf *g, int64_t i, x100_gguf_tensor *t);
int x100_gguf_find(const x100_gguf *g, const char *name, x100_gguf_tensor *t);

/* Metadata: key i in file order (name and value type; for arrays also the element type and
 * count), and typed getters by key.  A getter returns X100_ENOTFOUND when the key is absent or
 * has another type (the integer getter accepts every integer type whose value fits). */
int x100_gguf_kv_at(const x100_gguf *g, int64_t i, const char **key, uint32_t *type,
                    uint32_t *elem_type, uint64_t *count);
int x100_gguf_get_int(const x100_gguf *g, const char *key, int64_t *v);
int x100_gguf_get_float(const x100_gguf *g, const char *key, double *v);    /* F32 or F64 */
int x100_gguf_get_str(const x100_gguf *g, const char *key, const char **s, uint64_t *len);
/* Element j of a string array (e.g. tokenizer.ggml.tokens); s is not NUL-terminated. */
int x100_gguf_get_arr_str(const x100_gguf *g, const char *key, uint64_t j, const char **s, uint64_t *len);

int x100_gguf_qwen3moe_params(const x100_gguf *g, x100_gguf_qwen3moe *p);

/* ggml type name as bench/gguf_dump.c prints it ("Q4_K", ...; "?" for an unknown id), and the
 * bytes / elements of one block (0 / 0 for a type without a fixed block size here). */
const char *x100_gguf_type_name(uint32_t type);
size_t x100_gguf_block_bytes(uint32_t type);
int x100_gguf_block_elems(uint32_t type);

/* Copy bytes [byte0, byte0 + n) of a tensor's data to device memory dst on stream and wait for
 * the copy (the source is pageable memory of the mapping). */
int x100_gguf_upload(const x100_gguf *g, const x100_gguf_tensor *t, uint64_t byte0, uint64_t n, void *dst,
                     void *stream);

/* Rows [row0, row0 + n_rows) of a 2-D tensor (or of a 3-D expert tensor viewed as
 * dims[1]*dims[2] rows of dims[0] elements) uploaded and packed for qgemv_hip: w_packed must hold
 * x100q_packed_bytes(t->type, n_rows, dims[0]) bytes (256-byte aligned).  Q4_0, Q8_0, Q3_K,
 * Q4_K, Q5_K and Q6_K.  Synchronous (uses a temporary device buffer). */
int x100_gguf_pack_rows(const x100_gguf *g, const x100_gguf_tensor *t, uint64_t row0, uint64_t n_rows,
                        void *w_packed, void *stream);

#ifdef __cplusplus
}
#endif
#endif
