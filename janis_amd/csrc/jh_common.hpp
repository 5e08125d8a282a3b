// Internal declarations shared by the HIP sources of libjanis_hip.so.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <string>
#include <type_traits>

#include "../../include/janis_hip.h"

namespace jh {

// ---- element conversions --------------------------------------------------

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// float -> bfloat16, round to nearest even (NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

// Two floats -> packed bf16x2 (low half = a).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    return static_cast<uint32_t>(f32_to_bf16(a)) | (static_cast<uint32_t>(f32_to_bf16(b)) << 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// float -> IEEE half, round to nearest even (the hardware conversion).
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Raw buffer resources (gfx9 descriptor word 3 = 0x00020000: 32-bit dwords,
// no swizzle). A buffer load outside [0, bytes) returns 0 instead of faulting,
// and takes a 32-bit byte offset, so kernels address rows with 32-bit math and
// need no clamping. `bytes` must be below 2^31 (checked by the launchers).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
constexpr int kAuxNT = 2;  // non-temporal: streamed data, read once
// Device-coherent load (gfx950 sc1): misses the CU's L1 and is served by the
// XCD's L2, so it sees what another CU of the same XCD stored (a plain or sc0
// load may return the L1's stale copy; measured on MI355X).
constexpr int kAuxSc1 = 16;

__device__ __forceinline__ uint4 buf_load16_nt(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kAuxNT);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint16_t buf_load2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}

// fp32 -> bf16 bits with the hardware's round-to-nearest-even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint16_t f32_to_bf16_hw(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// 16-byte streaming load of packed weights (read once per call: non-temporal).
__device__ __forceinline__ uint4 load_stream16(const uint32_t* p) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Sum of v over each slice of LPR consecutive lanes (LPR a power of two <= 64),
// with DPP: an inclusive row_shr scan inside each row of 16 lanes, then
// row_bcast15/row_bcast31 to carry row totals across rows. The slice total is
// valid in the slice's LAST lane (lane % LPR == LPR - 1); other lanes hold
// partial sums.
template <int LPR>
__device__ __forceinline__ float slice_sum_last(float v) {
    auto dpp = [](float x, auto ctrl, auto row_mask) {
        return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                             0, __builtin_bit_cast(int, x), decltype(ctrl)::value,
                                             decltype(row_mask)::value, 0xF, false));
    };
    using C1 = std::integral_constant<int, 0x111>;  // row_shr:1
    using C2 = std::integral_constant<int, 0x112>;  // row_shr:2
    using C4 = std::integral_constant<int, 0x114>;  // row_shr:4
    using C8 = std::integral_constant<int, 0x118>;  // row_shr:8
    using B15 = std::integral_constant<int, 0x142>; // row_bcast:15
    using B31 = std::integral_constant<int, 0x143>; // row_bcast:31
    using All = std::integral_constant<int, 0xF>;
    if constexpr (LPR >= 2) v += dpp(v, C1{}, All{});
    if constexpr (LPR >= 4) v += dpp(v, C2{}, All{});
    if constexpr (LPR >= 8) v += dpp(v, C4{}, All{});
    if constexpr (LPR >= 16) v += dpp(v, C8{}, All{});
    if constexpr (LPR >= 32) v += dpp(v, B15{}, std::integral_constant<int, 0xA>{});
    if constexpr (LPR >= 64) v += dpp(v, B31{}, std::integral_constant<int, 0xC>{});
    return v;
}

// ---- wave reductions without LDS -------------------------------------------------
// DPP inside each row of 16 lanes (xor 1 and xor 2 inside quads, then the
// mirrors of 8 and of 16 lanes), then gfx950's v_permlane16_swap /
// v_permlane32_swap across rows: called with both operands v, the two results
// hold, in every lane, v of this lane and v of the lane 16 (32) away in the
// partner row (half), so their sum or max reduces over that pair. All VALU.
template <bool MAX>
__device__ __forceinline__ float row16_reduce(float v) {
    auto dpp = [](float x, auto ctrl) {
        return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x),
                                                                     decltype(ctrl)::value, 0xF, 0xF, false));
    };
    auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
    v = op(v, dpp(v, std::integral_constant<int, 0xB1>{}));   // quad_perm [1,0,3,2]
    v = op(v, dpp(v, std::integral_constant<int, 0x4E>{}));   // quad_perm [2,3,0,1]
    v = op(v, dpp(v, std::integral_constant<int, 0x141>{}));  // row_half_mirror
    v = op(v, dpp(v, std::integral_constant<int, 0x140>{}));  // row_mirror
    return v;
}
__device__ __forceinline__ float row16_sum(float v) { return row16_reduce<false>(v); }

template <bool MAX>
__device__ __forceinline__ float pair16(float v) {  // rows (0,1) and (2,3)
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return MAX ? fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1])) : __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
template <bool MAX>
__device__ __forceinline__ float pair32(float v) {  // halves (0-31, 32-63)
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return MAX ? fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1])) : __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// Over the 4 rows, per lane position in the row (result in every lane).
__device__ __forceinline__ float rows4_sum(float v) { return pair32<false>(pair16<false>(v)); }
__device__ __forceinline__ float rows4_max(float v) { return pair32<true>(pair16<true>(v)); }
// Over all 64 lanes (result in every lane).
__device__ __forceinline__ float wave_sum(float v) { return rows4_sum(row16_reduce<false>(v)); }
__device__ __forceinline__ float wave_max(float v) { return rows4_max(row16_reduce<true>(v)); }

// ---- 4-bit word dot products ------------------------------------------------------
// Codes become bf16 without conversion instructions: a code q in the low 4
// mantissa bits of bf16(128.0) = 0x4300 is exactly 128 + q. Two masks split a
// word into its even and odd codes (one per byte) and v_perm_b32 builds the bf16
// pairs (128 + q_p, 128 + q_{p+4}); v_dot2_f32_bf16 multiplies them with the
// input pairs (x_p, x_{p+4}) and accumulates in fp32. The 128 is removed per
// group through the input sum, either inside the dot product (the decode tiles
// start it from -128*sum(x)) or after it:
//   scale*sum(x*(128+q)) + (bias - 128*scale)*sum(x) = scale*sum(x*q) + bias*sum(x).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
constexpr uint32_t kBf16Bytes = 0x43434343u;  // 0x43 = high byte of bf16(128.0)
// v_perm_b32 selectors over {src0 = kBf16Bytes (bytes 4..7), src1 = codes (bytes 0..3)}:
// result bytes (low to high) = code byte 0, 0x43, code byte 2, 0x43  /  byte 1, 0x43, byte 3, 0x43
constexpr uint32_t kSelB0B2 = 0x04020400u;
constexpr uint32_t kSelB1B3 = 0x04030401u;
constexpr float kCodeOffset = 128.0f;

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), c, false);
}

// acc + sum_l (128 + q_l) * x_l over the 8 codes of `word`; xp[p] = (x_p, x_{p+4}).
// lo = word & 0x0F0F0F0F holds codes 0,2,4,6 one per byte, hi = (word >> 4) &
// 0x0F0F0F0F codes 1,3,5,7: 7 integer ops and 4 dot2 per word.
__device__ __forceinline__ float word_dot(uint32_t word, const uint32_t* xp, float acc) {
    const uint32_t lo = word & 0x0F0F0F0Fu;
    const uint32_t hi = (word >> 4) & 0x0F0F0F0Fu;
    acc = dot2_bf16(__builtin_amdgcn_perm(kBf16Bytes, lo, kSelB0B2), xp[0], acc);  // (q0, q4)
    acc = dot2_bf16(__builtin_amdgcn_perm(kBf16Bytes, hi, kSelB0B2), xp[1], acc);  // (q1, q5)
    acc = dot2_bf16(__builtin_amdgcn_perm(kBf16Bytes, lo, kSelB1B3), xp[2], acc);  // (q2, q6)
    acc = dot2_bf16(__builtin_amdgcn_perm(kBf16Bytes, hi, kSelB1B3), xp[3], acc);  // (q3, q7)
    return acc;
}

// The 8 bf16 inputs (x0,x1) (x2,x3) (x4,x5) (x6,x7) of one word regrouped as
// (x0,x4) (x1,x5) (x2,x6) (x3,x7); returns their fp32 sum, taken as the bf16
// pairs' dot products with (1, 1): four v_dot2_f32_bf16 instead of eight
// widenings and seven adds (the x preparation is a fixed cost per lane and
// block that a single-pass tile does not amortise).
constexpr uint32_t kBf16Ones = 0x3F803F80u;  // bf16 (1.0, 1.0)
__device__ __forceinline__ float pair_up(uint4 v, uint32_t* xp) {
    xp[0] = __builtin_amdgcn_perm(v.z, v.x, 0x05040100u);
    xp[1] = __builtin_amdgcn_perm(v.z, v.x, 0x07060302u);
    xp[2] = __builtin_amdgcn_perm(v.w, v.y, 0x05040100u);
    xp[3] = __builtin_amdgcn_perm(v.w, v.y, 0x07060302u);
    const float ab = dot2_bf16(v.y, kBf16Ones, dot2_bf16(v.x, kBf16Ones, 0.0f));
    const float cd = dot2_bf16(v.w, kBf16Ones, dot2_bf16(v.z, kBf16Ones, 0.0f));
    return ab + cd;
}

// Load element i of a scale/bias array of the given dtype as fp32 (exact).
__device__ __forceinline__ float load_sb(const void* p, int64_t i, int dt) {
    if (dt == JH_BF16) return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
    if (dt == JH_F16) return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
    return static_cast<const float*>(p)[i];
}

// fl32(fl32(q * s) + b): the product is rounded before the add, the order the
// reference's Dequantize computes on amd64 (cpu/cpu_misc.go:134-161);
// contraction into an FMA is switched off here (hipcc contracts by default).
__device__ __forceinline__ float unfused_qsb(float q, float s, float b) {
#pragma clang fp contract(off)
    const float p = q * s;
    return p + b;
}

__device__ __forceinline__ void store_y(void* y, int64_t i, float v, int dt) {
    if (dt == JH_BF16)
        static_cast<uint16_t*>(y)[i] = f32_to_bf16(v);
    else
        static_cast<float*>(y)[i] = v;
}

// ---- launch descriptors ------------------------------------------------------

// Slots of the sum-of-squares statistics a residual-add product hands to the
// next RMSNorm'd product (one partial per block, the rest zero).
constexpr int kNormSlots = JH_NORM_STATS;

struct QuantMatrix {
    const uint32_t* w;   // [rows, P]
    const void* scales;  // [rows, G]
    const void* biases;  // [rows, G]
    int sb_dtype;
    int64_t rows;        // out_features
    int64_t in;          // in_features (K)
    int group_size;
    int bits = 4;        // 2, 4 or 8: 32/bits codes per word
};

struct Status {
    int code = JH_OK;
    std::string msg;
    static Status ok() { return {}; }
    static Status fail(int c, std::string m) {
        Status s;
        s.code = c;
        s.msg = std::move(m);
        return s;
    }
};

// Launchers (return a failure only for launch-time errors).
Status launch_dequantize(const QuantMatrix& m, void* out, int out_dtype, hipStream_t st);
Status launch_qmv(const QuantMatrix& m, const void* x, int x_dtype, void* y, int y_dtype,
                  int num_cus, hipStream_t st);
// Decode product with a fused prologue (pro: 0 none, 1 RMSNorm of fp32 x with
// weight nw, 2 SiLU(x[:K]) * x[K:]) and epilogue (epi: 0 store, 1 y = resid +
// product in fp32, 2 SwiGLU over W = [gate rows; up rows], y has m.rows / 2).
struct NormSplit {
    float* stats = nullptr;    // kNormSlots fp32: read by prologue 3, written by epilogue 3
    uint16_t* out = nullptr;   // bf16 [rows]: epilogue 3's bf16(y * nw)
};
size_t qmv_fused_workspace_bytes(const QuantMatrix& m, int pro, int x_dtype, int nw_dtype, int epi, int y_dtype);
Status launch_qmv_fused(const QuantMatrix& m, int pro, const void* x, int x_dtype, const void* nw, int nw_dtype,
                        float eps, int epi, const float* resid, void* y, int y_dtype, const NormSplit& ns,
                        int num_cus, hipStream_t st, void* workspace);
// out = bf16(x * w), stats = the sum of x^2 in per-block partials (one row of d).
Status launch_norm_prepare(const void* x, int x_dt, int64_t d, const void* w, int w_dt, uint16_t* out, float* stats,
                           hipStream_t st);
// out = bf16(u / sqrt(sum(stats) / d + eps)).
Status launch_norm_apply(const uint16_t* u, int64_t d, const float* stats, float eps, uint16_t* out, hipStream_t st);
// What a launch that waits for other blocks of its own grid needs: zeroed
// counters (nullptr: no such launch), the poll bound and the host-visible
// status word a wait that gives up sets.
struct InLaunchSync {
    int* counters;
    uint32_t spin;
    int* status;
};
// A few bf16 or fp32 x rows (2..kQmvRowsMax; qmv_rows_ok says which calls, by
// rows, row length and matrix size) through the decode tiles, the weights read
// once per launch of 2, 4 or 8 rows.
constexpr int64_t kQmvRowsMax = 8;
bool qmv_rows_ok(const QuantMatrix& m, int64_t rows, int x_dtype);
Status launch_qmv_rows(const QuantMatrix& m, const void* x, int x_dtype, int64_t rows, void* y, int y_dtype,
                       int num_cus, hipStream_t st);
// `sync.counters` (the kQmmSyncSlot share, or nullptr) lets the split-K partial
// tiles be added inside the product's launch (see qmm.hip).
Status launch_qmm(const QuantMatrix& m, const void* x, int x_dtype, int64_t rows, void* y,
                  int y_dtype, int num_cus, hipStream_t st, void* workspace, InLaunchSync sync = {});
// fp32 accumulation buffer a split-K prefill needs (0 when none).
size_t qmm_workspace_bytes(const QuantMatrix& m, int64_t rows, int x_dtype, int y_dtype, int num_cus,
                           bool in_launch = false);

struct GatherArgs {
    QuantMatrix m;        // one expert's shape; w/scales/biases point at expert 0
    int64_t n_experts;
    const void* x;
    int x_dtype;
    int64_t n_lead, a_vectors, k_slots;
    const int32_t* idx;
    void* y;
    int y_dtype;
    void* workspace;      // gather_workspace_bytes(n_experts, n_lead*k_slots)
};
size_t gather_workspace_bytes(int64_t n_experts, int64_t n_pairs);
// False when the call buckets inside its product launch (no workspace needed).
bool gather_uses_workspace(const GatherArgs& a);
Status launch_gather(const GatherArgs& a, int num_cus, hipStream_t st);

// One MoE expert MLP over stacked experts: out = sum_k score * down(SiLU(gate x) * up x).
struct MoeMlpArgs {
    QuantMatrix gate, up, down;  // one expert's shapes; pointers at expert 0
    int64_t n_experts;
    const void* x;               // bf16 [n_tok, H]
    int64_t n_tok, k_slots;
    const int32_t* idx;          // [n_tok, k_slots]
    const float* scores;         // [n_tok, k_slots]
    void* out;                   // [n_tok, H]
    int out_dtype;
};
// ---- decode-step operators (decode.hip) ----
Status launch_rms_norm(const void* x, int x_dt, const void* w, int w_dt, float eps, void* out, int out_dt,
                       int64_t rows, int64_t d, hipStream_t st);
Status launch_rope(const void* x, int x_dt, void* out, int out_dt, int64_t rows, int64_t L, int64_t D, int dims,
                   bool traditional, float base, float scale, int64_t offset, const float* freqs, hipStream_t st);
bool sdpa_decode_ok(int q_dt, int kv_dt, int64_t Hq, int64_t Hk, int64_t Lq, int64_t Dh);
int64_t sdpa_splits(int64_t B, int64_t Hk, int64_t Lk, int num_cus);
size_t sdpa_workspace_bytes(int q_dt, int kv_dt, int64_t B, int64_t Hq, int64_t Hk, int64_t Lq, int64_t Lk,
                            int64_t Dh, int num_cus);
Status launch_sdpa(const void* q, int q_dt, const void* k, const void* v, int kv_dt, void* out, int out_dt,
                   int64_t B, int64_t Hq, int64_t Hk, int64_t Lq, int64_t Lk, int64_t kcap, int64_t Dh, float scale,
                   bool causal, void* workspace, int num_cus, hipStream_t st);
Status launch_elementwise(int op, const void* a, int a_dt, const void* b, int b_dt, void* out, int out_dt, int64_t n,
                          hipStream_t st);
size_t argmax_workspace_bytes(int64_t rows);
// With `sync` (the context's zeroed counters) rows up to kArgmaxSyncRows take
// one launch (the last block of a row merges its candidates); otherwise two.
Status launch_argmax(const void* x, int x_dt, int64_t rows, int64_t n, int32_t* out, void* workspace, int* sync,
                     hipStream_t st);
Status launch_qk_norm_rope_append(const void* qkv, int qkv_dt, int Hq, int Hk, const void* qn_w, const void* kn_w,
                                  int w_dt, float eps, float base, float scale, int64_t pos, void* kc, void* vc,
                                  int c_dt, int64_t cap, void* q_out, int q_dt, hipStream_t st);
// One-token attention (q/k norm, RoPE, KV append, SDPA over keys 0..pos): one
// launch, plus a merge launch when the keys are split over blocks.
size_t attn_decode_workspace_bytes(int64_t Hq, int64_t Hk, int64_t pos, int num_cus);
// `sync` (kAttnSyncSlots zeroed ints per context, or nullptr) lets the split
// partials be merged inside the attention launch when the GPU deals workgroups
// to its 8 XCDs round-robin (probe_xcd_round_robin) and the kv heads are a
// multiple of 8; otherwise a merge launch follows.
constexpr int kAttnSyncSlots = 4096 + 64 + 32 * 512;
// The fused q/k/v + attention launch's share of them: per XCD x, the arrival
// flags of its blocks at kAttnFlagSlot + 128 x (zero between calls).
constexpr int kAttnFlagSlot = 1024;
constexpr int kAttnMaxBlocksPerXcd = 128;
// jh_argmax's share: the arrival counter of row r at kArgmaxSyncSlot + r for
// the first kArgmaxSyncRows rows (zero between calls).
constexpr int kArgmaxSyncSlot = 2048, kArgmaxSyncRows = 2048;
// The fused launch's give-up markers, one per XCD (zero until a wait gives up;
// reset by the host, see jh_sync).
constexpr int kAttnMarkerSlot = 4096;
// The split-K prefill product's share: the arrival counter of output tile t at
// kQmmSyncSlot + 32 t (one 128-byte line each) for kQmmSyncTiles tiles (zero
// between calls).
constexpr int kQmmSyncSlot = 4096 + 64, kQmmSyncTiles = 512;
// Polls of the arrival flags before a fused launch's wait gives up (the default
// of jh_set_wait_limit).
constexpr uint32_t kDefaultWaitPolls = 1u << 22;
bool attn_merge_in_launch(int64_t Hk, const int* sync);
Status launch_attn_decode(const void* qkv, int qkv_dt, int Hq, int Hk, const void* qn_w, const void* kn_w, int w_dt,
                          float eps, float base, float rscale, const float* rope_cs, int64_t pos, void* kc,
                          void* vc, int c_dt, int64_t cap, float scale, void* out, int out_dt, void* workspace,
                          int num_cus, hipStream_t st, int* sync);
// The q/k/v product (JH_PRO_NORMED prologue, bf16 or f32 out) and the attention of one
// token in one launch (decode.hip); JH_ERR_UNSUPPORTED outside qkv_attn_ok.
bool qkv_attn_ok(const QuantMatrix& m, int64_t Hq, int64_t Hk, const int* sync, int num_cus);
Status launch_qkv_attn(const QuantMatrix& m, const uint16_t* x, float* stats, float norm_eps, void* qkv, int qkv_dt,
                       int Hq, int Hk, const void* qn_w, const void* kn_w, int w_dt, float eps, float base, float rscale,
                       const float* rope_cs, int64_t pos, void* kc, void* vc, int c_dt, int64_t cap, float scale,
                       void* out, int out_dt, void* workspace, int num_cus, hipStream_t st, int* sync,
                       uint32_t spin, int* status);
// 8 when block b of a launch runs on XCD b % 8 (checked on a 64-block launch;
// buf: 64 ints of device memory), else 0.
int probe_xcd_round_robin(int* buf, hipStream_t st);
Status launch_rope_table(int dims, float base, float scale, int64_t pos, const float* freqs, float* out,
                         hipStream_t st);
// Embedding row of ids[0] (4-bit, 2-bit or 8-bit codes) + the split RMSNorm
// producer half on it (+ the RoPE table at pos when cs is given), one launch.
Status launch_embed_norm(const int32_t* ids, const QuantMatrix& table, const void* w, int w_dt, float* h,
                         uint16_t* out, float* stats, int rope_dims, float base, float scale, int64_t pos, float* cs,
                         hipStream_t st);
constexpr int kMaxCopyDims = 8;
// dst = src over shape, both through element strides (dst_strides nullptr:
// contiguous), converting between F32/F16/BF16 (other types: same-type copies).
Status launch_copy_strided(const void* src, int sdt, int nd, const int64_t* shape, const int64_t* strides, void* dst,
                           int ddt, const int64_t* dst_strides, hipStream_t st);
// One batch of a row scatter: update row src[i] goes to row dst[i], i < n
// (passed by value, so a launch needs no device copy of the indices).
constexpr int kScatterBatch = 256;
constexpr int kScatterChunk = 64 * 1024;  // bytes of a row per block
struct ScatterList {
    int32_t dst[kScatterBatch];
    int32_t src[kScatterBatch];
    int n;
};
Status launch_scatter_rows(const ScatterList& l, const void* updates, void* out, int64_t row_bytes,
                           hipStream_t st);
Status launch_take_rows(const void* table, int64_t row_bytes, int64_t n_rows, const int32_t* ids, int64_t n_ids,
                        void* out, hipStream_t st);
Status launch_kv_append(void* kc, void* vc, int c_dt, const void* kn, const void* vn, int n_dt, int64_t BH,
                        int64_t cap, int64_t pos, int64_t L, int64_t Dh, hipStream_t st);

// Router: per token softmax over E logits, top-k, optional renormalisation.
Status launch_moe_route(const void* logits, int l_dt, int64_t n_tok, int E, int k, bool norm, int32_t* idx,
                        float* scores, hipStream_t st);
// Why the fused kernels cannot take this call, or nullptr.
const char* moe_unsupported(const MoeMlpArgs& a);
size_t moe_workspace_bytes(const MoeMlpArgs& a);
Status launch_moe_mlp(const MoeMlpArgs& a, void* workspace, hipStream_t st);

// ---- operators around the products (ops.hip) ----
// QuantMatmul with transpose = false: y [rows, m.in] = x [rows, m.rows] . Dequantize(W);
// with idx, the gather form over a stack of n_experts (rows = the slot pairs).
Status launch_quant_matmul_t(const QuantMatrix& m, const void* x, int x_dtype, int64_t rows, void* y, int y_dtype,
                             const int32_t* idx, int64_t n_experts, int64_t k_slots, int64_t a_vectors,
                             hipStream_t st);
// Softmax / Mean along the middle axis of an [outer, len, inner] view, fp32 out.
Status launch_softmax(const void* x, int x_dt, float* y, int64_t outer, int64_t len, int64_t inner, hipStream_t st);
Status launch_mean(const void* x, int x_dt, float* y, int64_t outer, int64_t len, int64_t inner, hipStream_t st);
Status launch_scalar(int op, const void* x, int x_dt, float v, void* y, int y_dt, int64_t n, hipStream_t st);
// res[0] += NaN/Inf count, res[1] = min(res[1], first index of one).
Status launch_nonfinite(const void* x, int x_dt, int64_t n, unsigned long long* res, hipStream_t st);

}  // namespace jh
