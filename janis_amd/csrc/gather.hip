// MoE expert product (GatherQuantMatmul, cpu/cpu_misc.go:178-230) on gfx950.
//
// The reference buckets the (lead, slot) pairs by expert on the host and runs
// one QuantMatmul per used expert. Here the bucketing runs on the device so the
// routing never has to come back to the host:
//
//  1. moe_bucket_kernel (one workgroup): counts the pairs per expert, lists the
//     used experts in ascending id order (the reference's iteration order),
//     and writes each expert's pairs in (lead, slot) order into a workspace:
//        ws[0]                  U, the number of used experts
//        ws[1 .. 1+E)           used expert ids
//        ws[1+E .. 2+2E)        bucket offsets (U+1 of them)
//        ws[2+2E .. 2+2E+pairs) pair ids  (pair = lead * k_slots + slot)
//     An out-of-range index gets a row of NaN and no bucket.
//  2. gather_qmv_kernel: grid (row blocks, min(E, pairs)); block (rb, u) loads
//     its rows of expert uniq[u] into registers ONCE and applies them to every
//     pair routed to that expert, so each used expert's packed weights are
//     read once per call and unused experts are never read. The inner product
//     is the decode kernel's: bf16 pairs (128+q) against bf16 x pairs with
//     v_dot2_f32_bf16, the 128 removed through the group's sum of x.
#include "jh_common.hpp"

namespace jh {

__global__ __launch_bounds__(256) void qmv_generic_kernel(
    const uint32_t* __restrict__ W, const void* __restrict__ S, const void* __restrict__ B,
    int sb_dt, const void* __restrict__ X, int x_dt, void* __restrict__ Y, int y_dt, int64_t N,
    int64_t K, int gs, int64_t M, const int* __restrict__ ws, int64_t n_experts,
    int64_t k_slots, int64_t a_vectors);

namespace {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
constexpr int kMaxExperts = 4096;

__global__ __launch_bounds__(1024) void moe_bucket_kernel(const int32_t* __restrict__ idx,
                                                          int64_t n_pairs, int64_t E,
                                                          int* __restrict__ ws,
                                                          void* __restrict__ Y, int y_dt,
                                                          int64_t N) {
    __shared__ int cnt[kMaxExperts];
    __shared__ int start[kMaxExperts];
    int* uniq = ws + 1;
    int* offs = ws + 1 + E;
    int* pairs = ws + 2 + 2 * E;
    for (int64_t e = threadIdx.x; e < E; e += blockDim.x) cnt[e] = 0;
    __syncthreads();
    for (int64_t p = threadIdx.x; p < n_pairs; p += blockDim.x) {
        const int e = idx[p];
        if (e >= 0 && e < E) {
            atomicAdd(&cnt[e], 1);
        } else {
            const float nan = __uint_as_float(0x7fc00000u);
            for (int64_t j = 0; j < N; j++) store_y(Y, p * N + j, nan, y_dt);
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int U = 0, off = 0;
        for (int64_t e = 0; e < E; e++) {
            start[e] = off;
            if (cnt[e] > 0) {
                uniq[U] = (int)e;
                offs[U] = off;
                off += cnt[e];
                U++;
            }
        }
        offs[U] = off;
        ws[0] = U;
    }
    __syncthreads();
    for (int64_t p = threadIdx.x; p < n_pairs; p += blockDim.x) {
        const int e = idx[p];
        if (e < 0 || e >= E) continue;
        int rank = 0;
        for (int64_t q = 0; q < p; q++) rank += (idx[q] == e);
        pairs[start[e] + rank] = (int)p;
    }
}

constexpr uint32_t kBf16Bytes = 0x43434343u;
constexpr uint32_t kSelB0B2 = 0x04020400u;
constexpr uint32_t kSelB1B3 = 0x04030401u;
constexpr float kCodeOffset = 128.0f;

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), c, false);
}

// acc + sum_l (128 + q_l) * x_l over the 8 codes of `word`; xa = x0..x7 as bf16
// pairs (x0,x1) (x2,x3) (x4,x5) (x6,x7). Codes become bf16 128 + q by placing
// them under the high byte 0x43 with v_perm_b32 (see qmv.hip); x is regrouped
// to (x_p, x_{p+4}) to match.
__device__ __forceinline__ float word_dot(uint32_t word, uint4 xa, float acc) {
    const uint32_t x04 = __builtin_amdgcn_perm(xa.z, xa.x, 0x05040100u);
    const uint32_t x15 = __builtin_amdgcn_perm(xa.z, xa.x, 0x07060302u);
    const uint32_t x26 = __builtin_amdgcn_perm(xa.w, xa.y, 0x05040100u);
    const uint32_t x37 = __builtin_amdgcn_perm(xa.w, xa.y, 0x07060302u);
    const uint32_t lo = word & 0x0F0F0F0Fu;
    const uint32_t hi = (word >> 4) & 0x0F0F0F0Fu;
    acc = dot2_bf16(__builtin_amdgcn_perm(kBf16Bytes, lo, kSelB0B2), x04, acc);
    acc = dot2_bf16(__builtin_amdgcn_perm(kBf16Bytes, hi, kSelB0B2), x15, acc);
    acc = dot2_bf16(__builtin_amdgcn_perm(kBf16Bytes, lo, kSelB1B3), x26, acc);
    acc = dot2_bf16(__builtin_amdgcn_perm(kBf16Bytes, hi, kSelB1B3), x37, acc);
    return acc;
}

__device__ __forceinline__ float sum8_bf16(uint4 v) {
    const float a = __uint_as_float(v.x << 16) + __uint_as_float(v.x & 0xFFFF0000u);
    const float b = __uint_as_float(v.y << 16) + __uint_as_float(v.y & 0xFFFF0000u);
    const float c = __uint_as_float(v.z << 16) + __uint_as_float(v.z & 0xFFFF0000u);
    const float d = __uint_as_float(v.w << 16) + __uint_as_float(v.w & 0xFFFF0000u);
    return (a + b) + (c + d);
}

template <bool SB_F16>
__device__ __forceinline__ float sb_at(const uint16_t* p, uint32_t i) {
    if constexpr (SB_F16)
        return f16_to_f32(p[i]);
    else
        return bf16_to_f32(p[i]);
}

// Rows per block = 4 waves * (64/LPR) slices * RPW rows. Loads use clamped row
// indices (always in bounds) and are issued back to back; stores are predicated.
template <int LPR, int ITERS, int RPW, bool SB_F16>
__global__ __launch_bounds__(256) void gather_qmv_kernel(
    const uint32_t* __restrict__ W, const uint16_t* __restrict__ S, const uint16_t* __restrict__ B,
    const uint16_t* __restrict__ X, void* __restrict__ Y, int y_dt, uint32_t N, int gs_log2,
    const int* __restrict__ ws, int64_t E, int64_t k_slots, int64_t a_vectors) {
    constexpr int SLICES = 64 / LPR;
    constexpr uint32_t P = 4 * LPR * ITERS;
    constexpr uint32_t K = 8 * P;
    const int U = ws[0];
    if ((int)blockIdx.y >= U) return;
    const int64_t e = ws[1 + blockIdx.y];
    const int p_begin = ws[1 + E + blockIdx.y], p_end = ws[2 + E + blockIdx.y];
    const int* pairs = ws + 2 + 2 * E;

    const int lane = threadIdx.x & 63;
    const int sl = lane % LPR, slice = lane / LPR;
    const uint32_t G = K >> gs_log2;
    const uint32_t row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * (SLICES * RPW) + slice * RPW;
    const uint32_t* We = W + e * (int64_t)N * P;
    const uint16_t* Se = S + e * (int64_t)N * G;
    const uint16_t* Be = B + e * (int64_t)N * G;

    uint4 wv[RPW][ITERS];
    float sc[RPW][ITERS], bo[RPW][ITERS];
#pragma unroll
    for (int r = 0; r < RPW; r++) {
        const uint32_t row = min(row0 + r, N - 1);
#pragma unroll
        for (int it = 0; it < ITERS; it++)
            wv[r][it] = load_stream16(We + (row * P + it * 4 * LPR + 4 * sl));
    }
#pragma unroll
    for (int r = 0; r < RPW; r++) {
        const uint32_t row = min(row0 + r, N - 1);
#pragma unroll
        for (int it = 0; it < ITERS; it++) {
            const uint32_t g = (32u * (it * LPR + sl)) >> gs_log2;
            const float s = sb_at<SB_F16>(Se, row * G + g);
            const float b = sb_at<SB_F16>(Be, row * G + g);
            sc[r][it] = s;
            bo[r][it] = fmaf(-kCodeOffset, s, b);
        }
    }

    for (int pi = p_begin; pi < p_end; pi++) {
        const int64_t pair = pairs[pi];
        const int64_t l = pair / k_slots, k = pair - l * k_slots;
        const int64_t xrow = l * a_vectors + (a_vectors == 1 ? 0 : k);
        const uint16_t* xr = X + xrow * K;
        float part[RPW];
#pragma unroll
        for (int r = 0; r < RPW; r++) part[r] = 0.0f;
#pragma unroll
        for (int it = 0; it < ITERS; it++) {
            const uint4* xv = reinterpret_cast<const uint4*>(xr + 32 * (it * LPR + sl));
            const uint4 x0 = xv[0], x1 = xv[1], x2 = xv[2], x3 = xv[3];
            const float xs = (sum8_bf16(x0) + sum8_bf16(x1)) + (sum8_bf16(x2) + sum8_bf16(x3));
#pragma unroll
            for (int r = 0; r < RPW; r++) {
                float d = 0.0f;
                d = word_dot(wv[r][it].x, x0, d);
                d = word_dot(wv[r][it].y, x1, d);
                d = word_dot(wv[r][it].z, x2, d);
                d = word_dot(wv[r][it].w, x3, d);
                part[r] = fmaf(sc[r][it], d, part[r]);
                part[r] = fmaf(bo[r][it], xs, part[r]);
            }
        }
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            const float v = slice_sum_last<LPR>(part[r]);
            const uint32_t row = row0 + r;
            if (sl == LPR - 1 && row < N) store_y(Y, pair * N + row, v, y_dt);
        }
    }
}

template <int LPR, int ITERS, int RPW, bool SB_F16>
Status run_fast_sb(const GatherArgs& a, int64_t max_u, int gs_log2, hipStream_t st) {
    constexpr int64_t rows_per_block = 4 * (64 / LPR) * RPW;
    const int64_t blocks = (a.m.rows + rows_per_block - 1) / rows_per_block;
    hipLaunchKernelGGL((gather_qmv_kernel<LPR, ITERS, RPW, SB_F16>), dim3((unsigned)blocks, (unsigned)max_u),
                       dim3(256), 0, st, a.m.w, static_cast<const uint16_t*>(a.m.scales),
                       static_cast<const uint16_t*>(a.m.biases), static_cast<const uint16_t*>(a.x),
                       a.y, a.y_dtype, (uint32_t)a.m.rows, gs_log2,
                       static_cast<const int*>(a.workspace), a.n_experts, a.k_slots, a.a_vectors);
    return Status::ok();
}

template <int LPR, int ITERS, int RPW>
Status run_fast(const GatherArgs& a, int64_t max_u, int gs_log2, hipStream_t st) {
    if (a.m.sb_dtype == JH_F16) return run_fast_sb<LPR, ITERS, RPW, true>(a, max_u, gs_log2, st);
    return run_fast_sb<LPR, ITERS, RPW, false>(a, max_u, gs_log2, st);
}

int log2_exact(int v) {
    int l = 0;
    while ((1 << l) < v) l++;
    return ((1 << l) == v) ? l : -1;
}

}  // namespace

size_t gather_workspace_bytes(int64_t n_experts, int64_t n_pairs) {
    return sizeof(int) * (size_t)(2 + 2 * n_experts + n_pairs);
}

Status launch_gather(const GatherArgs& a, int num_cus, hipStream_t st) {
    const int64_t n_pairs = a.n_lead * a.k_slots;
    if (n_pairs == 0) return Status::ok();
    if (a.n_experts > kMaxExperts)
        return Status::fail(JH_ERR_UNSUPPORTED, "gather_quant_matmul: more than 4096 experts");
    hipLaunchKernelGGL(moe_bucket_kernel, dim3(1), dim3(1024), 0, st, a.idx, n_pairs, a.n_experts,
                       static_cast<int*>(a.workspace), a.y, a.y_dtype, a.m.rows);
    const int64_t max_u = n_pairs < a.n_experts ? n_pairs : a.n_experts;
    if (max_u > 65535) return Status::fail(JH_ERR_UNSUPPORTED, "gather_quant_matmul: too many experts in one call");
    const int gl = log2_exact(a.m.group_size);
    const int64_t P = a.m.in / 8;
    const bool fast_ok = a.x_dtype == JH_BF16 && gl >= 5 && gl <= 7 && (a.m.in % a.m.group_size) == 0 &&
                         (a.m.sb_dtype == JH_BF16 || a.m.sb_dtype == JH_F16) &&
                         a.m.rows * (a.m.in / 8) < ((int64_t)1 << 32);
    if (fast_ok) {
        switch (P) {
            case 256 * 1: return run_fast<64, 1, 4>(a, max_u, gl, st);
            case 256 * 2: return run_fast<64, 2, 2>(a, max_u, gl, st);
            case 256 * 3: return run_fast<64, 3, 2>(a, max_u, gl, st);
            case 256 * 4: return run_fast<64, 4, 1>(a, max_u, gl, st);
            case 256 * 6: return run_fast<64, 6, 1>(a, max_u, gl, st);
            case 128 * 1: return run_fast<32, 1, 4>(a, max_u, gl, st);
            case 128 * 3: return run_fast<32, 3, 2>(a, max_u, gl, st);
            case 64 * 1: return run_fast<16, 1, 4>(a, max_u, gl, st);
            case 64 * 3: return run_fast<16, 3, 2>(a, max_u, gl, st);
            case 32 * 1: return run_fast<8, 1, 4>(a, max_u, gl, st);
            case 32 * 3: return run_fast<8, 3, 2>(a, max_u, gl, st);
            default: break;
        }
    }
    int64_t blocks = (a.m.rows + 3) / 4;
    const int64_t cap = (int64_t)num_cus * 4;
    if (blocks > cap) blocks = cap;
    hipLaunchKernelGGL(qmv_generic_kernel, dim3((unsigned)blocks, (unsigned)max_u), dim3(256), 0, st,
                       a.m.w, a.m.scales, a.m.biases, a.m.sb_dtype, a.x, a.x_dtype, a.y, a.y_dtype,
                       a.m.rows, a.m.in, a.m.group_size, (int64_t)0,
                       static_cast<const int*>(a.workspace), a.n_experts, a.k_slots, a.a_vectors);
    return Status::ok();
}

}  // namespace jh
