/*
 * janis_hip.h -- C ABI of the MI355X (gfx950) quantized-linear backend for
 * janis (github.com/guregodevo/janis).
 *
 * This is the boundary a cgo package would bind: plain pointers, sizes and
 * enums, no C++ or torch types. Each entry point names the method of janis's
 * engine.Backend interface (engine/backend.go) it implements. All tensor
 * pointers passed to the operator entry points are DEVICE pointers (from
 * jh_alloc or any other HIP allocation on the context's device), row-major and
 * contiguous. Operators are enqueued on the context's stream and return
 * without waiting; jh_d2h and jh_sync wait.
 *
 * Every function returns JH_OK (0) or a non-zero status; the message of the
 * last failure on a context is jh_last_error(ctx). The reference backends
 * panic on bad input (cpu/cpu_misc.go:137, ggml/ggml.go:439); a Go wrapper
 * turns a non-zero status into that panic.
 *
 * Threading: one context is used by one thread at a time, as janis drives its
 * backend from one engine thread (serve/serve.go:94-105). Distinct contexts are
 * independent.
 *
 * Workspace: operators that need device scratch memory (split-K prefill
 * partials, expert buckets, attention partials, argmax partials) take it from
 * one per-context workspace that grows on demand. A buffer the workspace grows
 * out of is kept until jh_destroy, so a HIP graph captured before the growth
 * still replays into valid memory; growth itself is refused (JH_ERR_INVALID)
 * while the context's stream is being captured, so make each captured call
 * once, eagerly, before the capture. Graphs captured on one context share its
 * workspace: replay them on one stream, not concurrently.
 */
#ifndef JANIS_HIP_H
#define JANIS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__) || defined(__clang__)
#define JH_API __attribute__((visibility("default")))
#else
#define JH_API
#endif

/* Element types; values equal engine.DType (engine/backend.go:11-21). */
typedef enum {
    JH_F32 = 0,
    JH_F16 = 1,
    JH_BF16 = 2,
    JH_I32 = 3,
    JH_U32 = 4,
    JH_U8 = 5
} jh_dtype;

/* Status codes. */
enum {
    JH_OK = 0,
    JH_ERR_INVALID = 1,     /* bad shape, dtype, pointer or argument */
    JH_ERR_UNSUPPORTED = 2, /* valid for the reference, not implemented here */
    JH_ERR_HIP = 3,         /* the HIP runtime reported an error */
    JH_ERR_OOM = 4,         /* device allocation failed */
    JH_ERR_NONFINITE = 5,   /* value checks on (JH_CHECK_VALUES): the result holds NaN/Inf */
    JH_ERR_TIMEOUT = 6      /* a launch that waits for its own blocks (jh_qkv_attention_decode, a
                               split-K jh_quant_matmul) gave up (reported by the next jh_sync /
                               jh_d2h / fused call / split-K call; see jh_set_wait_limit) */
};

typedef struct jh_ctx jh_ctx;

/* ---- context, memory, streams --------------------------------------------- */

/* Backend.Version (engine/backend.go:145): library name and version. */
JH_API const char *jh_version(void);

/* Creates a context on HIP device `device` with a stream of its own at the
 * default priority. Replaces the backend constructors ggml.New()
 * (ggml/ggml.go) and cpu.New() (cpu/cpu.go:84). */
JH_API int jh_create(int device, jh_ctx **out);

/* Backend.Close (engine/backend.go:286): waits for queued work, releases the
 * context's stream and workspace. Safe on NULL. */
JH_API void jh_destroy(jh_ctx *ctx);

/* Message of the last failure on ctx ("" if none). Valid until the next call
 * on ctx. With ctx == NULL, the last failure of jh_create. */
JH_API const char *jh_last_error(const jh_ctx *ctx);

/* Device name and compute-unit count, for EngineInfo (backend_cpu.go:27-30). */
JH_API int jh_device_info(jh_ctx *ctx, char *name, size_t name_len, int *compute_units);

/* Enqueue on a caller-owned hipStream_t instead of the context's own stream
 * (NULL restores the context's stream). The caller keeps the stream alive.
 * The exchanges inside one launch (the attention merges of
 * jh_attention_decode and jh_qkv_attention_decode, the split-K sums of
 * jh_quant_matmul's prefill product) need workgroups dealt to the 8 XCDs
 * round-robin, which jh_create checks; a stream whose CU mask leaves any CU out
 * (hipExtStreamCreateWithCUMask) runs them as separate launches instead. */
JH_API int jh_set_stream(jh_ctx *ctx, void *hip_stream);

/* Bound on the in-kernel waits, in polls: of jh_qkv_attention_decode's
 * attention blocks for the product blocks of their XCD, and of a split-K
 * prefill product's blocks for the other K splits of their output tile
 * (default 2^22, far beyond a normal wait of about a microsecond). When a wait
 * gives up, the outputs it guards are NaN (the call's attention output; the
 * product's rows of that block) and the next jh_sync / jh_d2h (or fused or
 * split-K call) returns JH_ERR_TIMEOUT and resets the synchronisation state.
 * 0 makes every wait give up at once: the failure path, for tests. No
 * counterpart in the reference: a safety bound of this backend's launches that
 * wait for their own blocks. */
JH_API int jh_set_wait_limit(jh_ctx *ctx, int64_t polls);

/* The hipStream_t operators are enqueued on. */
JH_API void *jh_get_stream(const jh_ctx *ctx);

/* Check flags of jh_set_checks. */
#define JH_CHECK_INDICES 1 /* device indices (expert ids, row ids) read back and range-checked */
#define JH_CHECK_VALUES 2  /* every float result read back and counted for NaN/Inf */

/* Read-back checks, the equivalent of janis's JANIS_GGML_CHECK
 * (ggml/ggml.go:622-677), off by default. flags is a combination of:
 *   JH_CHECK_INDICES  jh_gather_quant_matmul, jh_moe_swiglu and jh_take_rows
 *                     copy their indices to the host and reject an out-of-range
 *                     one with JH_ERR_INVALID before launching. When off, an
 *                     out-of-range expert index yields a row of NaN (a row id,
 *                     a row of zeros) and no memory outside the table is read.
 *   JH_CHECK_VALUES   after each operator with a float result (the quantized
 *                     products, the fused products, the decode-step operators,
 *                     Softmax/Mean/Scalar), the result is counted for NaN/Inf
 *                     on the device and any found is JH_ERR_NONFINITE naming
 *                     the operator, the count and the first index. The
 *                     reference reports the same and exits; here the caller
 *                     decides.
 * Both wait for the stream, so they refuse (JH_ERR_INVALID) a stream under
 * graph capture. jh_set_checks(ctx, 1) keeps its earlier meaning. */
JH_API int jh_set_checks(jh_ctx *ctx, int flags);

/* Counts the NaN/Inf among n device values of dtype (JH_F32, JH_BF16, JH_F16):
 * *count, and *first = the first index of one (n when none). Waits for the
 * stream. The check a caller can run on any tensor before Floats. */
JH_API int jh_check_finite(jh_ctx *ctx, const void *x, jh_dtype dtype, int64_t n, int64_t *count,
                           int64_t *first);

/* Waits for every operator enqueued on the context's stream. Returns
 * JH_ERR_TIMEOUT if a launch since the last check gave up its in-kernel wait
 * (see jh_set_wait_limit); jh_d2h does the same. */
JH_API int jh_sync(jh_ctx *ctx);

/* Device memory (hipMalloc / hipFree). jh_free(NULL) is a no-op. */
JH_API int jh_alloc(jh_ctx *ctx, size_t bytes, void **out);
JH_API int jh_free(jh_ctx *ctx, void *ptr);

/* Host -> device copy of `bytes`; returns once the source may be reused, as
 * FromRaw/FromFloats copy (engine/backend.go:147-154, mlxc/mlxc.go:27-31). */
JH_API int jh_h2d(jh_ctx *ctx, void *dst_device, const void *src_host, size_t bytes);

/* Device -> host copy after all queued work; the tail of Floats/Ints
 * (engine/backend.go:276-283). */
JH_API int jh_d2h(jh_ctx *ctx, void *dst_host, const void *src_device, size_t bytes);

/* Element-wise operators of jh_elementwise. */
typedef enum {
    JH_OP_ADD = 0,      /* a + b            Backend.Add  (cpu/cpu.go:300-302) */
    JH_OP_MUL = 1,      /* a * b            Backend.Mul  (cpu/cpu.go:304-306) */
    JH_OP_SILU = 2,     /* a / (1 + e^-a)   Backend.SiLU (cpu/cpu.go:327-329); b unused */
    JH_OP_SILU_MUL = 3  /* SiLU(a) * b      MLP.Forward's Mul(SiLU(gate), up) (qwen/mlp.go:33-35) */
} jh_op;

/* ---- MLX affine-quantized operators ---------------------------------------- *
 * Layout (MLX, cpu/cpu_misc.go:124-130): a quantized matrix of `rows` rows and
 * `in_features` columns is
 *   w       uint32 [rows, in_features * bits / 32], 32/bits codes per word,
 *           least-significant first;
 *   scales  [rows, in_features / group_size] of sb_dtype (JH_BF16, JH_F16 or JH_F32);
 *   biases  same shape and dtype as scales;
 * and element (r, j) is  scale * code + bias  with the group's scale and bias.
 * Supported here: bits 2, 4 and 8 (32/bits codes per word; other widths return
 * JH_ERR_UNSUPPORTED) and any group_size that divides in_features. 4-bit weights
 * with group sizes 32, 64 and 128 and bf16 activations take the fast kernels;
 * everything else a slower generic kernel.
 * w, x and y must be 16-byte aligned (jh_alloc gives 256). */

/* Backend.Dequantize (engine/backend.go:261-263; cpu/cpu_misc.go:134-161):
 * out[r, j] = fl32(code(r, j) * scale + bias), bit-identical to the CPU
 * backend, written as out_dtype (JH_F32, or JH_BF16 rounded to nearest-even). */
JH_API int jh_dequantize(jh_ctx *ctx, const uint32_t *w, const void *scales, const void *biases,
                  jh_dtype sb_dtype, int64_t rows, int64_t in_features, int group_size, int bits,
                  void *out, jh_dtype out_dtype);

/* Backend.QuantMatmul (engine/backend.go:265-267; cpu/cpu_misc.go:232-400).
 * transpose != 0 (the QuantizedLinear convention, the one the models use):
 *   y[rows, out_features] = x[rows, in_features] . W^T
 * transpose == 0 (the CPU backend's MatMul(x, Dequantize(w)), :233-236):
 *   y[rows, in_features] = x[rows, out_features] . Dequantize(W)
 *   with the CPU backend's order (each output a sum over the out_features rows
 *   in increasing order, terms rounded then added, zero x terms skipped), so its
 *   fp32 results have the CPU backend's bits; a slow path, off the models' path.
 * x_dtype and y_dtype are JH_BF16 or JH_F32; accumulation is fp32. rows == 1
 * runs the decode GEMV; a few rows run the decode GEMV's tiles with every
 * row's x in registers, so each row's result has the bits of a one-row call:
 * 2 rows always; 3..4 rows, except for in_features 768, 1536, 3072, 6144,
 * 12288 and 16384, where 3..4 rows take the tiles only from in_features 1536
 * with fewer than 2^24 weights (out_features x in_features); 5..8 rows with
 * in_features >= 1024 and fewer than 2^24 weights (where those tiles are the
 * faster path on MI355X). Other row counts run the MFMA prefill GEMM. rows == 0
 * is a no-op. fp32 x (the activation type
 * of the CPU backend, of Dequantize and of the embedding) takes the same tiles:
 * each lane rounds its part of x to bf16 (nearest even) in registers, so an
 * fp32-x call has the bits of a bf16-x call on bf16(x). Shapes outside the
 * tiles run a generic kernel that multiplies fp32 x unrounded.
 * When the prefill GEMM splits K, its fp32 partial products go to the
 * context's workspace (grown to split * rows * out_features floats) and are
 * added in a fixed order: results are the same bits on every call. Where the
 * product's blocks all fit on the GPU at once, the sums are made inside its
 * launch, whose blocks then wait for each other (bounded: jh_set_wait_limit);
 * split-K calls on one GPU must then be serialised and not run beside kernels
 * that hold its CUs, as for jh_qkv_attention_decode. The GEMM
 * multiplies x rounded to bf16: fp32 x is first rounded into the workspace
 * (rows * in_features bf16 more), so fp32 x gives the bits of its bf16
 * rounding passed as bf16. */
JH_API int jh_quant_matmul(jh_ctx *ctx, const void *x, jh_dtype x_dtype, int64_t rows, const uint32_t *w,
                    const void *scales, const void *biases, jh_dtype sb_dtype, int64_t out_features,
                    int64_t in_features, int transpose, int group_size, int bits, void *y,
                    jh_dtype y_dtype);

/* Backend.GatherQuantMatmul (engine/backend.go:269-274; cpu/cpu_misc.go:178-230),
 * the MoE expert product. transpose != 0:
 *   x            [n_lead, a_vectors, in_features]  (the reference's [lead.., A, 1, in]);
 *                a_vectors == 1 shares one vector across the k_slots experts,
 *                a_vectors == k_slots gives each slot its own vector;
 *   w/scales/biases stacked over experts: [n_experts, out_features, .];
 *   rhs_indices  int32 [n_lead, k_slots], device memory;
 *   y            [n_lead, k_slots, out_features]   (the reference's [lead.., K, 1, out]).
 * Slots are bucketed by expert on the device, so each routed expert's packed
 * weights are read once per call whatever the number of slots routed to it,
 * and experts nobody routed to are not read. One call = one bucketing launch
 * plus one product launch.
 * transpose == 0: each slot is the transposed product of jh_quant_matmul with
 * its expert's matrix (cpu/cpu_misc.go:224 with :233-236): x [n_lead,
 * a_vectors, out_features], y [n_lead, k_slots, in_features]. (The reference
 * sizes that result's rows by the stack's out_features, which agrees when the
 * experts are square.) */
JH_API int jh_gather_quant_matmul(jh_ctx *ctx, const void *x, jh_dtype x_dtype, int64_t n_lead,
                           int64_t a_vectors, const uint32_t *w, const void *scales,
                           const void *biases, jh_dtype sb_dtype, int64_t n_experts,
                           int64_t out_features, int64_t in_features, const int32_t *rhs_indices,
                           int64_t k_slots, int transpose, int group_size, int bits, void *y,
                           jh_dtype y_dtype);

/* ---- the other operators of a decode step ---------------------------------- *
 * Activations are JH_BF16 or JH_F32 (norm weights also JH_F16); arithmetic is
 * fp32 with exp/sqrt/cos/sin/pow in double as the CPU backend evaluates them.
 * All pointers are device memory. */

/* Backend.RMSNorm (engine/backend.go; cpu/cpu_ops.go:144-162) over rows of d:
 * out = x / sqrt(mean(x^2) + eps) * w. */
JH_API int jh_rms_norm(jh_ctx *ctx, const void *x, jh_dtype x_dtype, int64_t rows, int64_t d,
                const void *w, jh_dtype w_dtype, float eps, void *out, jh_dtype out_dtype);

/* Backend.RoPE / RoPEFreqs (cpu/cpu_attn.go:13-62): x holds rows of D features,
 * the row's position is offset + (row % L); the first `dims` features rotate
 * (traditional: pairs (2i, 2i+1), else (i, i+dims/2)) by pos*scale*inv_i with
 * inv_i = base^(-2i/dims), or 1/freqs[i] when freqs (fp32 [dims/2]) is given. */
JH_API int jh_rope(jh_ctx *ctx, const void *x, jh_dtype x_dtype, int64_t rows, int64_t L, int64_t D,
            int dims, int traditional, float base, float scale, int64_t offset, const float *freqs,
            void *out, jh_dtype out_dtype);

/* Backend.SDPA (cpu/cpu_attn.go:64-119): q [B, Hq, Lq, Dh]; k, v laid out as
 * [B, Hk, kv_capacity, Dh] with the first Lk rows valid (a KV cache, or
 * kv_capacity == Lk for plain tensors); GQA (head h reads kv head h/(Hq/Hk));
 * causal masks keys past (Lk - Lq) + i for query row i. out [B, Hq, Lq, Dh].
 * k/v are JH_BF16, JH_F16 (what KVCache.Update's cast makes, qwen/cache.go:
 * 90-93) or JH_F32. Lq == 1 with bf16 or f16 k/v, Dh == 128 and Hq/Hk in
 * {1,2,4,8} runs split over the
 * keys (flash-decoding); other shapes a per-row kernel. */
JH_API int jh_sdpa(jh_ctx *ctx, const void *q, jh_dtype q_dtype, const void *k, const void *v,
            jh_dtype kv_dtype, int64_t B, int64_t Hq, int64_t Hk, int64_t Lq, int64_t Lk,
            int64_t kv_capacity, int64_t Dh, float scale, int causal, void *out, jh_dtype out_dtype);

/* Backend.Add / Mul / SiLU and the SwiGLU product, over n elements of equal
 * shape (b ignored for JH_OP_SILU). */
JH_API int jh_elementwise(jh_ctx *ctx, jh_op op, const void *a, jh_dtype a_dtype, const void *b,
                   jh_dtype b_dtype, int64_t n, void *out, jh_dtype out_dtype);

/* Backend.Argmax over the last axis (cpu/cpu_misc.go:91-121): the first index
 * of the maximum of each of `rows` rows of n; int32 out. */
JH_API int jh_argmax(jh_ctx *ctx, const void *x, jh_dtype x_dtype, int64_t rows, int64_t n, int32_t *out);

/* RowScatterer.ScatterRows (engine/backend.go:95-105; CPU semantics
 * cpu/cpu_ops.go:215-233): out = dst with out[indices[i]] = updates[i] along
 * the leading axis, for a dst of `rows` rows of row_bytes bytes and updates of
 * n_indices rows. indices are host memory, as the interface passes them; a
 * repeated index keeps the last of its updates; an index outside [0, rows) is
 * JH_ERR_INVALID, before anything is written. out == dst updates in place;
 * any other out (rows * row_bytes, not overlapping dst) receives a copy of dst
 * first. */
JH_API int jh_scatter_rows(jh_ctx *ctx, const void *dst, void *out, int64_t rows, int64_t row_bytes,
                           const int32_t *indices, int64_t n_indices, const void *updates);

/* The data movement behind Slice, Transpose, Concat, Cast and making a view
 * contiguous (engine/backend.go: Slice, Transpose, Concat, Cast; CPU semantics
 * cpu/cpu.go, cpu/cpu_misc.go): for every index of shape[ndim] (ndim <= 8),
 * dst[index . dst_strides] = src[index . src_strides] (strides in elements, any
 * sign, zero for broadcast; dst_strides NULL: dst contiguous), converted
 * between JH_F32 / JH_F16 / JH_BF16 (round to nearest even); JH_I32 / JH_U32 /
 * JH_U8 copy only to their own type. */
JH_API int jh_copy_strided(jh_ctx *ctx, const void *src, jh_dtype src_dtype, int ndim, const int64_t *shape,
                    const int64_t *src_strides, void *dst, jh_dtype dst_dtype, const int64_t *dst_strides);

/* Backend.TakeAxis on axis 0 (cpu/cpu_misc.go:48-89) for any element type:
 * out[i] = table row ids[i] (row_bytes each); ids is int32, device. An id
 * outside [0, n_rows) gives a zero row (JH_ERR_INVALID with checks on). With
 * Dequantize this is QuantEmbedding.Forward (qwen/embed.go:78-83). */
JH_API int jh_take_rows(jh_ctx *ctx, const void *table, int64_t row_bytes, int64_t n_rows,
                 const int32_t *ids, int64_t n_ids, void *out);

/* KV-cache append (the KVAppender capability, engine/backend.go:56-61; the
 * reference KVCache.Update, qwen/cache.go:90): writes k_new/v_new
 * [BH, L, Dh] into rows pos .. pos+L-1 of the caches [BH, capacity, Dh].
 * Caches and new rows are JH_BF16, JH_F16 or JH_F32 (converted, nearest even):
 * KVCache.Update casts f32 keys and values to f16 on a backend that reports
 * dtypes (qwen/cache.go:90-93). */
JH_API int jh_kv_append(jh_ctx *ctx, void *k_cache, void *v_cache, jh_dtype cache_dtype, int64_t BH,
                 int64_t capacity, int64_t pos, const void *k_new, const void *v_new,
                 jh_dtype new_dtype, int64_t L, int64_t Dh);

/* The middle of Attention.ForwardCached for one token (qwen/attention.go:101-122)
 * in one launch, for a backend that offers it: from the token's q/k/v product
 * [(n_heads + 2 n_kv_heads) * head_dim] (q heads, then k, then v), each query
 * head is RMS-normalised with q_norm_w and rotated (non-traditional RoPE,
 * inv_i = rope_base^(-2i/head_dim), angle pos * rope_scale * inv_i) into q_out
 * [n_heads, head_dim]; each key head normalised with k_norm_w, rotated and
 * written to row pos of k_cache [n_kv_heads, capacity, head_dim]; each value
 * head copied to row pos of v_cache. Same arithmetic as jh_rms_norm + jh_rope +
 * jh_kv_append. head_dim must be 128. */
JH_API int jh_qk_norm_rope_append(jh_ctx *ctx, const void *qkv, jh_dtype qkv_dtype, int64_t n_heads,
                           int64_t n_kv_heads, int64_t head_dim, const void *q_norm_w,
                           const void *k_norm_w, jh_dtype w_dtype, float eps, float rope_base,
                           float rope_scale, int64_t pos, void *k_cache, void *v_cache,
                           jh_dtype cache_dtype, int64_t capacity, void *q_out, jh_dtype q_out_dtype);

/* Attention.ForwardCached for one new token (qwen/attention.go:98-128) after
 * the q/k/v product, in one launch, for a backend that offers it: the work of
 * jh_qk_norm_rope_append (per-head q/k RMSNorm when q_norm_w/k_norm_w are given,
 * non-traditional RoPE at pos, the new key and value rows written to row pos of
 * the caches) followed by jh_sdpa over keys 0..pos (Lq = 1, one query row per
 * head), with the same arithmetic. The new key and value enter the softmax as
 * the bf16 values written to the cache. One launch when the cache is short;
 * longer ones split the keys over blocks, which write partial softmaxes to the
 * context's workspace for a second, merging launch.
 *   qkv       [(n_heads + 2 n_kv_heads) * 128]: q heads, then k heads, then v heads
 *   rope_cs   NULL, or jh_rope_table(128, rope_base, rope_scale, pos) (the same
 *             factors, computed once for all layers)
 *   caches    bf16 or f16 [n_kv_heads, capacity, 128] (cache_dtype); pos < capacity
 *   out       [n_heads * 128] (the input of the o product)
 * head_dim must be 128, n_heads / n_kv_heads 1, 2, 4 or 8. */
JH_API int jh_attention_decode(jh_ctx *ctx, const void *qkv, jh_dtype qkv_dtype, int64_t n_heads,
                        int64_t n_kv_heads, int64_t head_dim, const void *q_norm_w,
                        const void *k_norm_w, jh_dtype w_dtype, float eps, float rope_base,
                        float rope_scale, const float *rope_cs, int64_t pos, void *k_cache,
                        void *v_cache, jh_dtype cache_dtype, int64_t capacity, float scale, void *out,
                        jh_dtype out_dtype);

/* The q/k/v product of one token and its attention in one launch: exactly
 * jh_quant_matvec_fused(JH_PRO_NORMED, x, norm_stats, norm_eps, w/scales/biases
 * with (n_heads + 2 n_kv_heads) * head_dim rows, JH_EPI_STORE, y = qkv of
 * qkv_dtype bf16 or f32) followed by jh_attention_decode(qkv, qkv_dtype, ...),
 * with the same results bit
 * for bit: Attention.Forward's QuantLinear calls, QNorm/KNorm, RoPE, the KV
 * append and SDPA of one token (qwen/attention.go:98-128) after the block's
 * input RMSNorm (qwen/block.go:59). An optional capability in the pattern of
 * engine/backend.go:38-112 (the reference makes these calls one by one).
 * On MI355X with 8 kv heads, head_dim 128, in_features 4096 and 4-bit codes in
 * groups of 64 with bf16 scales, the kv head h's rows are computed on XCD h and
 * its attention follows there in the same launch (workgroups are dealt to the
 * XCDs round-robin; jh_create checks this); any other call runs the two
 * operators. The fused launch's attention blocks wait, inside the kernel, for
 * the product blocks of their XCD; the launch is sized so that all its blocks
 * are resident at once, so the wait ends when the GPU's CUs are free for it.
 * Fused calls on one GPU must therefore be serialised (one stream, or calls
 * ordered by the caller) and must not run beside kernels that hold the CUs
 * indefinitely. The wait is bounded (jh_set_wait_limit): a wait that gives up
 * makes the call's attention output NaN and is reported as JH_ERR_TIMEOUT by
 * the next jh_sync, jh_d2h or fused call, never silently. */
JH_API int jh_qkv_attention_decode(jh_ctx *ctx, const void *x, const float *norm_stats, float norm_eps,
                                   const uint32_t *w, const void *scales, const void *biases, jh_dtype sb_dtype,
                                   int64_t in_features, int group_size, int bits, void *qkv,
                                   jh_dtype qkv_dtype, int64_t n_heads,
                                   int64_t n_kv_heads, int64_t head_dim, const void *q_norm_w,
                                   const void *k_norm_w, jh_dtype w_dtype, float eps, float rope_base,
                                   float rope_scale, const float *rope_cs, int64_t pos, void *k_cache,
                                   void *v_cache, jh_dtype cache_dtype, int64_t capacity, float scale, void *out,
                                   jh_dtype out_dtype);

/* jh_attention_decode for callers that cannot allocate device memory (code
 * under HIP graph capture on a context whose workspace was never sized, tight
 * serving loops, harnesses that forbid hipMalloc). It has no counterpart in the
 * reference. Same arguments, arithmetic and results (bit for bit) as
 * jh_attention_decode, but the split partials go to a fixed 4 MiB device array
 * of the library (one per GPU, held until the process ends) instead of the
 * context's workspace, and nothing is allocated. The partials take
 * n_kv_heads * splits * (n_heads / n_kv_heads) * 130 floats, and the split
 * count is bounded by the CU count, so on a 256-CU MI355X every call fits (at
 * most ~3.2 MiB: 3 * CUs * 8 * 130 floats); a call that needs more than the
 * array (a part with more CUs) returns JH_ERR_UNSUPPORTED. Every call on one
 * GPU shares that array, from any
 * context: calls that overlap on one GPU (other streams, other threads) race
 * and must be ordered by the caller. No value checks (JH_CHECK_VALUES) run here. */
JH_API int jh_attention_decode_noalloc(jh_ctx *ctx, const void *qkv, jh_dtype qkv_dtype, int64_t n_heads,
                                       int64_t n_kv_heads, int64_t head_dim, const void *q_norm_w,
                                       const void *k_norm_w, jh_dtype w_dtype, float eps, float rope_base,
                                       float rope_scale, const float *rope_cs, int64_t pos, void *k_cache,
                                       void *v_cache, jh_dtype cache_dtype, int64_t capacity, float scale,
                                       void *out, jh_dtype out_dtype);

/* The RoPE factors at one position, for callers that rotate many heads there
 * (the RoPE angles of cpu/cpu_attn.go:13-34): out[i] = cos(theta_i) and
 * out[dims/2 + i] = sin(theta_i), theta_i = pos * scale * inv_i, inv_i =
 * base^(-2i/dims) or 1/freqs[i] (freqs fp32 [dims/2], may be NULL); pow, cos
 * and sin in double, rounded to fp32, as jh_rope evaluates them. out is fp32
 * [dims], device. Computed once per decode step, it serves every layer's
 * jh_attention_decode (rope_cs), which otherwise evaluates them in each block. */
JH_API int jh_rope_table(jh_ctx *ctx, int dims, float base, float scale, int64_t pos, const float *freqs,
                  float *out);

/* The router of MoEBlock.Forward (qwen/moe.go:455-491) on the device, for a
 * backend that offers it: per token, softmax over the n_experts logits
 * (cpu/cpu.go:461-499), the k largest by the reference's selection sort
 * (qwen/moe.go:420-444, ties as it breaks them), and with norm_topk != 0 the k
 * scores divided by their sum (NormTopk, :472-481). The reference copies the
 * probabilities to the host for this (the per-layer sync at :459); here the
 * indices and scores stay on the device for jh_moe_swiglu or
 * jh_gather_quant_matmul. Bit-identical to the CPU backend: the same fp32 order
 * of operations and exp evaluated in double.
 *   logits       [n_tok, n_experts] of logits_dtype (JH_F32 or JH_BF16), device
 *   rhs_indices  int32 [n_tok, k] (global expert ids), device
 *   scores       fp32 [n_tok, k], device
 * n_experts up to 4096. */
JH_API int jh_moe_route(jh_ctx *ctx, const void *logits, jh_dtype logits_dtype, int64_t n_tok,
                 int64_t n_experts, int64_t k, int norm_topk, int32_t *rhs_indices, float *scores);

/* The expert MLP of moeApply (qwen/moe.go:501-511) in one call, for a backend
 * that offers it (the engine's optional-capability pattern,
 * engine/backend.go:38-112). The reference composes it from three
 * GatherQuantMatmul calls and four element-wise operators:
 *   g = gather(x, gate), u = gather(x, up)      one vector per token (A = 1)
 *   h = SiLU(g) * u                              SiLU(v) = v / (1 + exp(-v))
 *   d = gather(h, down)                          one vector per slot (A = k_slots)
 *   out[t, :] = mean_k(d[t, k, :] * scores[t, k]) * k_slots
 * Here it is two launches: gate+up with the SiLU*mul epilogue (h stays on the
 * device in bf16), then the down product with the score-weighted sum taken in
 * a fixed order (slot order, then a fixed tree of four partial sums) and
 * written once; calls of more than 32 (token, slot) pairs add a bucketing
 * launch and a launch that sums each token's weighted slot rows in slot order.
 * No atomics: repeated calls give the same bits.
 *   x            bf16 [n_tok, hidden] (x_dtype must be JH_BF16)
 *   gate, up     stacked [n_experts, intermediate, hidden * bits / 32] with
 *                scales/biases [n_experts, intermediate, hidden / group_size]
 *   down         stacked [n_experts, hidden, intermediate * bits / 32] with
 *                scales/biases [n_experts, hidden, intermediate / group_size]
 *   rhs_indices  int32 [n_tok, k_slots] and scores fp32 [n_tok, k_slots], device memory
 *   out          [n_tok, hidden] of out_dtype (JH_F32 or JH_BF16)
 * A token with an index outside [0, n_experts)
 * gets a row of NaN (or JH_ERR_INVALID when jh_set_checks is on). Shapes
 * outside the expert tiles (hidden and intermediate in {256, 512, 768, 1024,
 * 1536, 2048, 3072, 4096, 6144, 8192, 12288}, group_size 32/64/128, 16-bit
 * scales shared by the three stacks) return JH_ERR_UNSUPPORTED; callers then
 * compose it from jh_gather_quant_matmul as the reference does. */
JH_API int jh_moe_swiglu(jh_ctx *ctx, const void *x, jh_dtype x_dtype, int64_t n_tok,
                  const uint32_t *w_gate, const void *s_gate, const void *b_gate,
                  const uint32_t *w_up, const void *s_up, const void *b_up,
                  const uint32_t *w_down, const void *s_down, const void *b_down,
                  jh_dtype sb_dtype, int64_t n_experts, int64_t hidden, int64_t intermediate,
                  const int32_t *rhs_indices, const float *scores, int64_t k_slots,
                  int group_size, int bits, void *out, jh_dtype out_dtype);

/* Backend.Softmax (engine/backend.go:241-242; cpu/cpu.go:461-499) along the
 * middle axis of x viewed as [outer, len, inner] (axis a of a shape d: outer =
 * d0..d(a-1), len = d(a), inner = d(a+1)..): the maximum, e = exp(x - max) in
 * double rounded to fp32, e / sum(e), with the CPU backend's sequential fp32
 * sum for len <= 8192 (bit-identical; longer lines sum in a tree). y is fp32
 * of x's shape. The router softmax of MoEBlock.Forward (qwen/moe.go:458). */
JH_API int jh_softmax(jh_ctx *ctx, const void *x, jh_dtype x_dtype, int64_t outer, int64_t len, int64_t inner,
                      float *y);

/* Backend.Mean (engine/backend.go:186; cpu/cpu_ops.go:113-142) over the middle
 * axis of [outer, len, inner]: y [outer, inner] fp32, each the sequential fp32
 * sum along the axis divided by len (bit-identical to the CPU backend). */
JH_API int jh_mean(jh_ctx *ctx, const void *x, jh_dtype x_dtype, int64_t outer, int64_t len, int64_t inner,
                   float *y);

/* Backend.ScalarMul / ScalarAdd (engine/backend.go:250-252; cpu/cpu_misc.go:24-30). */
typedef enum {
    JH_SCALAR_MUL = 0, /* y = x * v */
    JH_SCALAR_ADD = 1  /* y = x + v */
} jh_scalar_op;
JH_API int jh_scalar(jh_ctx *ctx, jh_scalar_op op, const void *x, jh_dtype x_dtype, int64_t n, float v, void *y,
                     jh_dtype y_dtype);

/* Prologues and epilogues of jh_quant_matvec_fused. */
typedef enum {
    JH_PRO_NONE = 0,     /* x_in = x */
    JH_PRO_RMSNORM = 1,  /* x_in = RMSNorm(x, norm_w, eps): Block.ForwardCached's InputNorm /
                            PostNorm feeding q/k/v and gate/up (qwen/block.go:59-60), and the
                            final norm feeding the LM head (qwen/model.go:294-303) */
    JH_PRO_SILU_MUL = 2, /* x holds [gate | up] (2 * in_features): x_in = SiLU(gate) * up,
                            MLP.Forward's input to Down (qwen/mlp.go:33-35) */
    JH_PRO_NORMED = 3    /* the same RMSNorm, prepared by the producer of x: x is the bf16
                            norm_out and norm_stats the statistics that a JH_EPI_RESID_NORM
                            call (or jh_norm_prepare) wrote; the product is scaled by
                            1 / sqrt(sum(norm_stats) / in_features + eps) */
} jh_prologue;

typedef enum {
    JH_EPI_STORE = 0,    /* y = x_in . W^T */
    JH_EPI_RESID = 1,    /* y = resid + x_in . W^T in fp32 (y_dtype JH_F32; resid may be y):
                            the residual adds of Block.ForwardCached (qwen/block.go:59-60) */
    JH_EPI_SWIGLU = 2,   /* W holds 2 * out_features rows, the Gate rows then the Up rows
                            (scales/biases likewise): y[j] = SiLU(g_j) * u_j with
                            g = x_in . Gate^T, u = x_in . Up^T in fp32 (MLP.Forward's
                            Mul(SiLU(Gate.Forward(x)), Up.Forward(x)), qwen/mlp.go:33-35) */
    JH_EPI_RESID_NORM = 3 /* JH_EPI_RESID, and the input of the NEXT RMSNorm'd product:
                            norm_out = bf16(y * norm_w) with norm_w that norm's weight
                            [out_features], and norm_stats (JH_NORM_STATS fp32) the sum of
                            y^2 split in partials; pass both to that product with
                            JH_PRO_NORMED */
} jh_epilogue;

/* fp32 slots of the statistics buffer of JH_EPI_RESID_NORM / JH_PRO_NORMED. */
#define JH_NORM_STATS 1024

/* One decode product with the operators on either side of it, for a backend
 * that offers it (the engine's optional-capability pattern,
 * engine/backend.go:38-112). It replaces the reference's sequences
 *   RMSNorm -> QuantMatmul                 (prologue JH_PRO_RMSNORM)
 *   Mul(SiLU(gate), up) -> QuantMatmul      (prologue JH_PRO_SILU_MUL)
 *   QuantMatmul -> Add(resid, .)            (epilogue JH_EPI_RESID)
 *   QuantMatmul(Gate), QuantMatmul(Up) -> Mul(SiLU(.), .)  (epilogue JH_EPI_SWIGLU)
 * for one row (rows == 1 of jh_quant_matmul, transpose = true):
 *   x_in = bf16(prologue(x))  (as jh_rms_norm / jh_elementwise with a bf16 out)
 *   the product with fp32 accumulation (as jh_quant_matmul), then the epilogue.
 * On the one-launch path RMSNorm is applied as (bf16(x * norm_w) . W^T) /
 * sqrt(mean(x^2) + eps): the same value up to where the bf16 rounding of the
 * product's input falls (the product is linear in it), with no reduction
 * ahead of the weight stream.
 * One launch where the decode tiles take the shape (4-bit weights, group size
 * 32/64/128, bf16 scales, K = in_features in {256, 512, 768, 1024, 1536, 2048,
 * 3072, 4096, 6144, 8192, 12288, 16384}) and
 *   JH_PRO_NONE with JH_EPI_STORE or JH_EPI_RESID, x bf16, or
 *   JH_PRO_RMSNORM with JH_EPI_STORE or JH_EPI_SWIGLU, x fp32, norm_w bf16:
 * each block normalises its own copy of x in registers (no normalised copy
 * goes through HBM) and the add or SwiGLU happens in the product's epilogue.
 * Everything else runs the same arithmetic as separate launches through the
 * context's workspace.
 *   x       [in_features] ([2 * in_features] for JH_PRO_SILU_MUL), device
 *   resid   fp32 [out_features] for JH_EPI_RESID / JH_EPI_RESID_NORM, else ignored
 *   y       [out_features] of y_dtype
 *   norm_stats, norm_out   for JH_PRO_NORMED (stats in) and JH_EPI_RESID_NORM
 *           (stats and bf16 [out_features] out); a call cannot use both
 * The split RMSNorm (JH_EPI_RESID_NORM then JH_PRO_NORMED) moves the x * w part
 * of the norm into the epilogue of the product that makes x, so the product
 * that consumes it reads bf16 x like a plain one: y = (bf16(x * w) . W^T) /
 * sqrt(mean(x^2) + eps), with mean(x^2) summed from per-block partials in a
 * fixed order. It needs the one-launch tiles (and bf16 norm weights); other
 * shapes run as jh_norm_prepare-style and separate launches. */
JH_API int jh_quant_matvec_fused(jh_ctx *ctx, jh_prologue prologue, const void *x, jh_dtype x_dtype,
                          const void *norm_w, jh_dtype norm_w_dtype, float eps, const uint32_t *w,
                          const void *scales, const void *biases, jh_dtype sb_dtype,
                          int64_t out_features, int64_t in_features, int group_size, int bits,
                          jh_epilogue epilogue, const float *resid, void *y, jh_dtype y_dtype,
                          float *norm_stats, void *norm_out);

/* The producer half of a split RMSNorm for a row the caller already holds (the
 * embedding row that enters the first block): norm_out = bf16(x * norm_w) [d]
 * and norm_stats (JH_NORM_STATS fp32) = the sum of x^2 in partials (the rest 0), for a
 * jh_quant_matvec_fused call with JH_PRO_NORMED. */
JH_API int jh_norm_prepare(jh_ctx *ctx, const void *x, jh_dtype x_dtype, int64_t d, const void *norm_w,
                    jh_dtype norm_w_dtype, void *norm_out, float *norm_stats);

/* The decode step's entry into the first block, one launch: h = the embedding
 * row of token ids[0] (QuantEmbedding.Forward, qwen/embed.go:78-83: TakeAxis of
 * the packed table, its scales and biases, then Dequantize, cpu/cpu_misc.go:
 * 134-161; zeros for an id outside [0, vocab), as jh_take_rows gives), then
 * jh_norm_prepare on h with norm_w (the first block's InputNorm), and, when
 * rope_cs is not NULL, jh_rope_table(rope_dims, rope_base, rope_scale, pos)
 * into rope_cs. Every output is bit-identical to those separate calls.
 *   ids      int32 [1], device (the previous step's jh_argmax output)
 *   w/scales/biases  the [vocab, dims] table (bits 2, 4 or 8)
 *   h        F32 [dims]; norm_out bf16 [dims]; norm_stats JH_NORM_STATS fp32
 * No counterpart call in the reference: it fuses the three its decode step makes
 * (qwen/model.go:294-303 embedding, qwen/block.go:58 InputNorm, and the RoPE
 * factors every Attention.ForwardCached call evaluates). */
JH_API int jh_embed_norm_prepare(jh_ctx *ctx, const int32_t *ids, const uint32_t *w, const void *scales,
                          const void *biases, jh_dtype sb_dtype, int64_t vocab, int64_t dims,
                          int group_size, int bits, const void *norm_w, jh_dtype norm_w_dtype,
                          float *h, void *norm_out, float *norm_stats, int rope_dims, float rope_base,
                          float rope_scale, int64_t pos, float *rope_cs);

#ifdef __cplusplus
}
#endif
#endif /* JANIS_HIP_H */
