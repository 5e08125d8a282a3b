// Decode GEMV for MLX affine 4-bit weights on gfx950:  y[n] = sum_k x[k] * W[n,k].
//
// Reference semantics: QuantMatmul with rows == 1 (cpu/cpu_misc.go:257-276),
// whose AVX2 kernel (cpu/qmv_amd64.s:28-81) factors each group as
//   scale_g * sum(x*q) + bias_g * sum(x).
// This kernel keeps that factorisation and maps it onto CDNA4:
//
//  * Rows are served by "slices" of LPR lanes (LPR = 64 for K >= 2048, fewer for
//    short rows so one wave covers several rows). Lane l of a slice owns a fixed
//    set of 32-element runs of the row, so its part of x is loaded ONCE per wave
//    into registers and reused for every row the wave visits.
//  * Each lane streams its words with 128-bit loads; a slice reads LPR*16
//    contiguous bytes per row and iteration (coalesced).
//  * Nibbles become bf16 with one AND-OR: (w >> 4p) & 0x000F000F | 0x43004300 is
//    the bf16 pair (128 + q_p, 128 + q_{p+4}), exact. v_dot2_f32_bf16 multiplies
//    it with the bf16 pair (x_p, x_{p+4}) and accumulates in fp32, so 8 codes
//    cost 7 integer ops and 4 dot2. The constant 128 is removed per group
//    through the x-sum that the factorisation needs anyway:
//      scale*sum(x*(128+q)) + (bias - 128*scale)*sum(x) = scale*sum(x*q) + bias*sum(x).
//  * Partial sums are reduced across the slice with cross-lane adds; the
//    slice's first lane writes y (fp32 or bf16).
#include "jh_common.hpp"

namespace jh {
namespace {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

constexpr uint32_t kNibPair = 0x000F000Fu;
constexpr uint32_t kBf16Base = 0x43004300u;  // bf16(128.0) in both halves
constexpr float kCodeOffset = 128.0f;

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), c, false);
}

// acc + sum_l (128 + q_l) * x_l over the 8 codes of `word`; xp[p] = (x_p, x_{p+4}).
__device__ __forceinline__ float word_dot(uint32_t word, const uint32_t* xp, float acc) {
    acc = dot2_bf16((word & kNibPair) | kBf16Base, xp[0], acc);
    acc = dot2_bf16(((word >> 4) & kNibPair) | kBf16Base, xp[1], acc);
    acc = dot2_bf16(((word >> 8) & kNibPair) | kBf16Base, xp[2], acc);
    acc = dot2_bf16(((word >> 12) & kNibPair) | kBf16Base, xp[3], acc);
    return acc;
}

// The 8 bf16 inputs of one word, (x0..x7) in 4 dwords, regrouped as the pairs
// (x0,x4) (x1,x5) (x2,x6) (x3,x7); returns their fp32 sum.
__device__ __forceinline__ float pair_up(uint4 v, uint32_t* xp) {
    xp[0] = (v.x & 0xFFFFu) | (v.z << 16);
    xp[1] = (v.x >> 16) | (v.z & 0xFFFF0000u);
    xp[2] = (v.y & 0xFFFFu) | (v.w << 16);
    xp[3] = (v.y >> 16) | (v.w & 0xFFFF0000u);
    const float a = __uint_as_float(v.x << 16) + __uint_as_float(v.x & 0xFFFF0000u);
    const float b = __uint_as_float(v.y << 16) + __uint_as_float(v.y & 0xFFFF0000u);
    const float c = __uint_as_float(v.z << 16) + __uint_as_float(v.z & 0xFFFF0000u);
    const float d = __uint_as_float(v.w << 16) + __uint_as_float(v.w & 0xFFFF0000u);
    return (a + b) + (c + d);
}

template <int LPR>
__device__ __forceinline__ float slice_sum(float v) {
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// LPR lanes per row, ITERS 128-bit loads per lane per row (K = 256*LPR*ITERS/... ):
//   words per row P = 4 * LPR * ITERS.  RPW rows per slice per pass.
template <int LPR, int ITERS, int RPW>
__global__ __launch_bounds__(256) void qmv_bf16x_kernel(
    const uint32_t* __restrict__ W, const void* __restrict__ S, const void* __restrict__ B,
    int sb_dt, const uint16_t* __restrict__ X, void* __restrict__ Y, int y_dt, int64_t N,
    int gs_log2) {
    constexpr int SLICES = 64 / LPR;
    constexpr int64_t P = 4 * LPR * ITERS;
    const int lane = threadIdx.x & 63;
    const int sl = lane % LPR;
    const int slice = lane / LPR;
    const int64_t G = (P * 8) >> gs_log2;

    uint32_t xp[ITERS][16];
    float xs[ITERS];
    int gi[ITERS];
#pragma unroll
    for (int it = 0; it < ITERS; it++) {
        const int e0 = 32 * (it * LPR + sl);
        const uint4* xv = reinterpret_cast<const uint4*>(X + e0);
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) s += pair_up(xv[j], &xp[it][4 * j]);
        xs[it] = s;
        gi[it] = e0 >> gs_log2;
    }

    const int64_t wave = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int64_t nwaves = (int64_t)gridDim.x * (blockDim.x >> 6);
    constexpr int ROWS_PER_WAVE = SLICES * RPW;

    for (int64_t base = wave * ROWS_PER_WAVE; base < N; base += nwaves * ROWS_PER_WAVE) {
        const int64_t row0 = base + (int64_t)slice * RPW;
        uint4 wv[RPW][ITERS];
        float sc[RPW][ITERS], bo[RPW][ITERS];
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            const int64_t row = row0 + r;
            const bool ok = row < N;
            const uint32_t* wr = W + row * P + 4 * sl;
#pragma unroll
            for (int it = 0; it < ITERS; it++) {
                if (ok) {
                    wv[r][it] = load_stream16(wr + it * 4 * LPR);
                    const float s = load_sb(S, row * G + gi[it], sb_dt);
                    const float b = load_sb(B, row * G + gi[it], sb_dt);
                    sc[r][it] = s;
                    bo[r][it] = fmaf(-kCodeOffset, s, b);
                } else {
                    wv[r][it] = make_uint4(0, 0, 0, 0);
                    sc[r][it] = 0.0f;
                    bo[r][it] = 0.0f;
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            float part = 0.0f;
#pragma unroll
            for (int it = 0; it < ITERS; it++) {
                float d = 0.0f;
                d = word_dot(wv[r][it].x, &xp[it][0], d);
                d = word_dot(wv[r][it].y, &xp[it][4], d);
                d = word_dot(wv[r][it].z, &xp[it][8], d);
                d = word_dot(wv[r][it].w, &xp[it][12], d);
                part = fmaf(sc[r][it], d, part);
                part = fmaf(bo[r][it], xs[it], part);
            }
            part = slice_sum<LPR>(part);
            const int64_t row = row0 + r;
            if (sl == 0 && row < N) store_y(Y, row, part, y_dt);
        }
    }
}

}  // namespace

// Generic kernel: any x dtype (bf16/f32), any K % 8 == 0 and group size dividing
// K, several x rows. One wave per output row; lane p handles words p, p+64, ...
// and dequantizes each code as fma(q, scale, bias) (== fl32(q*scale+bias) for
// bf16/f16 scales) before the fp32 dot, like the prefill path of the reference
// (cpu/cpu_misc.go:378-399). It also serves the gather product when `ws` holds
// an expert bucketing (see gather.hip): then blockIdx.y selects the bucket.
__global__ __launch_bounds__(256) void qmv_generic_kernel(
    const uint32_t* __restrict__ W, const void* __restrict__ S, const void* __restrict__ B,
    int sb_dt, const void* __restrict__ X, int x_dt, void* __restrict__ Y, int y_dt, int64_t N,
    int64_t K, int gs, int64_t M, const int* __restrict__ ws, int64_t n_experts,
    int64_t k_slots, int64_t a_vectors) {
    const int lane = threadIdx.x & 63;
    const int64_t P = K >> 3, G = K / gs;
    int64_t e = 0, p_begin = 0, p_end = M;
    const int* pairs = nullptr;
    if (ws) {
        const int U = ws[0];
        if ((int64_t)blockIdx.y >= U) return;
        const int* uniq = ws + 1;
        const int* offs = ws + 1 + n_experts;
        pairs = ws + 2 + 2 * n_experts;
        e = uniq[blockIdx.y];
        p_begin = offs[blockIdx.y];
        p_end = offs[blockIdx.y + 1];
    }
    const uint32_t* We = W + e * N * P;
    const int64_t sb0 = e * N * G;
    const int64_t wave = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int64_t nwaves = (int64_t)gridDim.x * (blockDim.x >> 6);
    for (int64_t row = wave; row < N; row += nwaves) {
        for (int64_t pi = p_begin; pi < p_end; pi++) {
            int64_t xrow = pi, yrow = pi;
            if (ws) {
                const int64_t pair = pairs[pi];
                const int64_t l = pair / k_slots, k = pair % k_slots;
                xrow = l * a_vectors + (a_vectors == 1 ? 0 : k);
                yrow = pair;
            }
            float part = 0.0f;
            for (int64_t p = lane; p < P; p += 64) {
                const uint32_t word = We[row * P + p];
#pragma unroll
                for (int l = 0; l < 8; l++) {
                    const int64_t j = 8 * p + l;
                    const int64_t g = j / gs;
                    const float s = load_sb(S, sb0 + row * G + g, sb_dt);
                    const float b = load_sb(B, sb0 + row * G + g, sb_dt);
                    const float w = fmaf((float)((word >> (4 * l)) & 0xFu), s, b);
                    const float xv = (x_dt == JH_BF16)
                                         ? bf16_to_f32(static_cast<const uint16_t*>(X)[xrow * K + j])
                                         : static_cast<const float*>(X)[xrow * K + j];
                    part = fmaf(xv, w, part);
                }
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) part += __shfl_xor(part, o, 64);
            if (lane == 0) store_y(Y, yrow * N + row, part, y_dt);
        }
    }
}

namespace {

template <int LPR, int ITERS, int RPW>
Status run_fast(const QuantMatrix& m, const void* x, void* y, int y_dtype, int gs_log2,
                int num_cus, hipStream_t st) {
    constexpr int64_t rows_per_block = 4 * (64 / LPR) * RPW;
    int64_t blocks = (m.rows + rows_per_block - 1) / rows_per_block;
    const int64_t cap = (int64_t)num_cus * 8;
    if (blocks > cap) blocks = cap;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL((qmv_bf16x_kernel<LPR, ITERS, RPW>), dim3((unsigned)blocks), dim3(256), 0,
                       st, m.w, m.scales, m.biases, m.sb_dtype,
                       static_cast<const uint16_t*>(x), y, y_dtype, m.rows, gs_log2);
    return Status::ok();
}

int log2_exact(int v) {
    int l = 0;
    while ((1 << l) < v) l++;
    return ((1 << l) == v) ? l : -1;
}

}  // namespace

Status launch_generic(const QuantMatrix& m, const void* x, int x_dtype, int64_t rows, void* y,
                      int y_dtype, int num_cus, hipStream_t st) {
    int64_t blocks = (m.rows + 3) / 4;
    const int64_t cap = (int64_t)num_cus * 16;
    if (blocks > cap) blocks = cap;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(qmv_generic_kernel, dim3((unsigned)blocks, 1), dim3(256), 0, st, m.w,
                       m.scales, m.biases, m.sb_dtype, x, x_dtype, y, y_dtype, m.rows, m.in,
                       m.group_size, rows, nullptr, (int64_t)1, (int64_t)1, (int64_t)1);
    return Status::ok();
}

Status launch_qmv(const QuantMatrix& m, const void* x, int x_dtype, void* y, int y_dtype,
                  int num_cus, hipStream_t st) {
    const int gl = log2_exact(m.group_size);
    const int64_t P = m.in / 8;
    const bool fast_ok = x_dtype == JH_BF16 && gl >= 5 && gl <= 7 && (m.in % m.group_size) == 0;
    if (fast_ok) {
        switch (P) {
            case 256 * 1: return run_fast<64, 1, 4>(m, x, y, y_dtype, gl, num_cus, st);
            case 256 * 2: return run_fast<64, 2, 4>(m, x, y, y_dtype, gl, num_cus, st);
            case 256 * 3: return run_fast<64, 3, 2>(m, x, y, y_dtype, gl, num_cus, st);
            case 256 * 4: return run_fast<64, 4, 2>(m, x, y, y_dtype, gl, num_cus, st);
            case 256 * 6: return run_fast<64, 6, 1>(m, x, y, y_dtype, gl, num_cus, st);
            case 256 * 8: return run_fast<64, 8, 1>(m, x, y, y_dtype, gl, num_cus, st);
            case 128 * 1: return run_fast<32, 1, 4>(m, x, y, y_dtype, gl, num_cus, st);
            case 128 * 3: return run_fast<32, 3, 2>(m, x, y, y_dtype, gl, num_cus, st);
            case 64 * 1: return run_fast<16, 1, 4>(m, x, y, y_dtype, gl, num_cus, st);
            case 64 * 3: return run_fast<16, 3, 2>(m, x, y, y_dtype, gl, num_cus, st);
            case 32 * 1: return run_fast<8, 1, 4>(m, x, y, y_dtype, gl, num_cus, st);
            case 32 * 3: return run_fast<8, 3, 2>(m, x, y, y_dtype, gl, num_cus, st);
            default: break;
        }
    }
    return launch_generic(m, x, x_dtype, 1, y, y_dtype, num_cus, st);
}

}  // namespace jh
