/*
 * janis_oracle.h -- TEST INFRASTRUCTURE ONLY.
 *
 * A CPU restatement, in plain C, of the arithmetic of janis's pure-Go CPU
 * backend for the MLX affine-quantized matrix products (module
 * github.com/guregodevo/janis). It is the checker the HIP backend is compared
 * against and the CPU baseline bench.py times. Nothing in the product
 * (janis_amd/) links, loads or calls it; only tests/, the smoke check in
 * __graft_entry__.py and bench.py's cpu_baseline leg do.
 *
 * Every function names the reference file:line whose arithmetic it follows,
 * including the order of floating-point operations where that order is part of
 * the reference's result (lane mapping, fused vs unfused multiply-adds,
 * reduction trees). All arithmetic is IEEE fp32 with round-to-nearest-even;
 * the translation unit is compiled with -ffp-contract=off so that only the
 * explicit fmaf() calls fuse.
 *
 * Conventions (cpu/cpu_misc.go:124-130, cpu/cpu.go:168-202):
 *   W      [rows, P]  uint32, 32/bits codes per word, least-significant first
 *   S, B   [rows, G]  fp32 (bf16 on disk, widened exactly by <<16)
 *   in   = P * 32/bits input features, G = in / group_size
 *   code(r, j) = (W[r, j / vpw] >> ((j % vpw) * bits)) & (2^bits - 1)
 *
 * Parity status of each function is recorded next to it; every function here
 * is pinned by at least one check in tests/test_oracle.py.
 */
#ifndef JANIS_ORACLE_H
#define JANIS_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Dequantize: out[r, j] = fl32(fl32(code * S[r, g]) + B[r, g]), g = j / gs.
 * Follows cpu/cpu_misc.go:134-161 (unfused multiply then add, as Go compiles
 * it on amd64). */
void or_dequantize(const uint32_t *w, const float *s, const float *b, float *out,
                   int64_t rows, int64_t P, int64_t G, int group_size, int bits);

/* qChannel4Ref (cpu/qmv_test.go:11-29): one 4-bit output channel, scalar,
 * element order, every product rounded before its add. */
float or_qchannel4_ref(const uint32_t *w, const float *x, const float *s, const float *b,
                       int groups, int words_per_group);

/* qChannel4AVX2 (cpu/qmv_amd64.s:28-81) restated lane by lane in scalar C:
 * lane l (0..7) takes code l of every word and x[8p+l];
 *   sumXQ_l = fma(q, x, sumXQ_l); sumX_l = sumX_l + x         (per word)
 *   acc_l   = fma(S_g, sumXQ_l, acc_l); acc_l = fma(B_g, sumX_l, acc_l)  (per group)
 *   result  = ((l0+l4)+(l1+l5)) + ((l2+l6)+(l3+l7)).
 * This is the bit-exact target; or_qchannel4_avx2 must equal it. */
float or_qchannel4_avx2_order(const uint32_t *w, const float *x, const float *s, const float *b,
                              int groups, int words_per_group);

/* The same kernel written with AVX2/FMA intrinsics (the CPU baseline that
 * bench.py times). Returns NaN if the host lacks AVX2+FMA; check
 * or_have_avx2_fma() first. */
float or_qchannel4_avx2(const uint32_t *w, const float *x, const float *s, const float *b,
                        int groups, int words_per_group);
int or_have_avx2_fma(void);

/* The portable decode path of QuantMatmul for 4-bit rows==1
 * (cpu/cpu_misc.go:277-347): 4-channel register blocking inside each
 * parallel chunk, 2-lane remainder. Chunking follows parallelFor
 * (cpu/cpu.go:37-62) with `workers` chunks, gated by parWork
 * (cpu/cpu.go:69-79). */
void or_qmv_blocked_go(const float *x, const uint32_t *w, const float *s, const float *b,
                       float *y, int64_t N, int64_t K, int group_size, int workers);

/* The generic-width decode path (cpu/cpu_misc.go:350-375), any bits. */
void or_qmv_generic(const float *x, const uint32_t *w, const float *s, const float *b,
                    float *y, int64_t N, int64_t K, int group_size, int bits);

/* The prefill path (rows > 1, cpu/cpu_misc.go:378-399): per output channel
 * wbuf[i] = fl32(fl32(q*S)+B), then acc = acc + x[i]*wbuf[i] sequentially. */
void or_qmm_wbuf(const float *x, int64_t rows, const uint32_t *w, const float *s, const float *b,
                 float *y, int64_t N, int64_t K, int group_size, int bits);

/* QuantMatmul with transpose=true as dispatched on an amd64 host
 * (cpu/cpu_misc.go:232-400): rows == 1 && gs % vpw == 0 && bits == 4 takes
 * the per-channel AVX2 kernel when simd != 0 (quant4SIMD, cpu/qmv_amd64.go:10-15),
 * else the blocked path; other widths take the generic decode path; rows > 1
 * takes the wbuf path. x is [rows, K], y is [rows, N]. `simd`=1 uses
 * or_qchannel4_avx2_order, so the result does not depend on the host ISA. */
void or_quant_matmul(const float *x, int64_t rows, const uint32_t *w, const float *s,
                     const float *b, float *y, int64_t N, int64_t K, int group_size, int bits,
                     int simd);

/* GatherQuantMatmul (cpu/cpu_misc.go:178-230). x is [n_lead, A, in]
 * (A == 1 shares one vector across the k_slots slots, A == k_slots gives one
 * per slot), w/s/b are stacked [E, N, .], idx is [n_lead, k_slots], y is
 * [n_lead, k_slots, N]. (lead, slot) pairs are bucketed by expert in
 * lead-major order and each used expert runs one or_quant_matmul with R rows
 * (R == 1 takes the decode path, R > 1 the wbuf path). Returns 0, or -1 if an
 * index lies outside [0, E) (the reference panics there). */
int or_gather_quant_matmul(const float *x, int64_t n_lead, int64_t A, const uint32_t *w,
                           const float *s, const float *b, int64_t E, const int32_t *idx,
                           int64_t k_slots, float *y, int64_t N, int64_t K, int group_size,
                           int bits, int simd);

/* Multi-threaded decode QuantMatmul for the CPU baseline: rows split into
 * `workers` contiguous chunks as parallelFor does (cpu/cpu.go:37-62), each
 * channel computed by the AVX2 kernel (or its scalar restatement when the
 * host lacks AVX2). Returns the number of worker threads used. */
int or_qmv_avx2_parallel(const float *x, const uint32_t *w, const float *s, const float *b,
                         float *y, int64_t N, int64_t K, int group_size, int workers);

/* moeApply (qwen/moe.go:501-511) with resident stacks and global expert ids:
 *   g = gather(x, gate), u = gather(x, up)          (A = 1: one vector per token)
 *   h = SiLU(g) * u, SiLU(v) = v / (1 + fl32(exp(-v)))   (cpu/cpu.go:327-329, :304-306)
 *   d = gather(h, down)                              (A = k_slots)
 *   out[t, :] = fl32(fl32(sum_k d[t,k,:]*score[t,k]) / K) * K   (cpu/cpu_ops.go:113-142, cpu/cpu_misc.go:24-26)
 * x [n_tok, H], stacks gate/up [E, I, H/8] and down [E, H, I/8] (4-bit), idx and
 * scores [n_tok, K], out [n_tok, H]. Returns 0, or -1 on an index out of range. */
int or_moe_apply(const float *x, int64_t n_tok, const uint32_t *wg, const float *sg,
                 const float *bg, const uint32_t *wu, const float *su, const float *bu,
                 const uint32_t *wd, const float *sd, const float *bd, int64_t E, int64_t H,
                 int64_t I, const int32_t *idx, const float *scores, int64_t k_slots, float *out,
                 int group_size, int simd);

/* Router top-k (qwen/moe.go:420-444): selection sort on a copy of the index
 * order, strict '>' comparison, k passes; writes idx[k], val[k]. */
void or_topk(const float *row, int n, int k, int32_t *idx, float *val);

/* Softmax along a row (cpu/cpu.go:461-499): max-subtract, exp in double
 * rounded to float, fp32 running sum, divide. */
void or_softmax_row(const float *x, float *out, int n);

/* ---- decode-step operators (engine.Backend methods of the CPU backend) ---- */

/* RMSNorm (cpu/cpu_ops.go:144-162) over rows of d. */
void or_rms_norm(const float *x, const float *w, float *out, int64_t rows, int64_t d, float eps);

/* RoPE / RoPEFreqs (cpu/cpu_attn.go:13-62); freqs may be NULL. */
void or_rope(const float *x, float *out, int64_t rows, int64_t L, int64_t D, int dims, int traditional,
             float base, float scale, int64_t offset, const float *freqs);

/* SDPA (cpu/cpu_attn.go:64-119), GQA and the offset causal mask. */
void or_sdpa(const float *q, const float *k, const float *v, float *out, int64_t B, int64_t Hq, int64_t Hk,
             int64_t Lq, int64_t Lk, int64_t Dh, float scale, int causal);

/* SiLU (cpu/cpu.go:327-329). */
void or_silu(const float *x, float *out, int64_t n);

/* Argmax over the last axis (cpu/cpu_misc.go:91-121). */
void or_argmax(const float *x, int64_t rows, int64_t n, int32_t *out);

#ifdef __cplusplus
}
#endif
#endif
