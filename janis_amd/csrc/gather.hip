// MoE expert product (GatherQuantMatmul, cpu/cpu_misc.go:178-230) on gfx950.
//
// The reference buckets the (lead, slot) pairs by expert on the host and runs
// one QuantMatmul per used expert. Here the bucketing runs on the device, so the
// routing never comes back to the host, and each routed expert's packed weights
// are read once per call whatever the number of slots routed to it:
//
//  * decode-sized calls (pairs <= kFusedMaxPairs): ONE launch. Every block
//    stages the indices in LDS, marks the used experts in a bitmap, takes the
//    u-th used expert (ascending id, the reference's iteration order) for
//    blockIdx.y = u and collects that expert's pairs; then it loads its rows of
//    the expert into registers and applies them to each pair.
//  * larger calls: moe_bucket_kernel writes the buckets to a workspace
//        ws[0]                  U, the number of used experts
//        ws[1 .. 1+E)           used expert ids, ascending
//        ws[1+E .. 2+2E)        bucket offsets (U+1 of them)
//        ws[2+2E .. 2+2E+pairs) pair ids (pair = lead * k_slots + slot)
//    and the product kernel reads them.
// An out-of-range index gets a row of NaN and no bucket. The inner product is
// the decode GEMV's: bf16 pairs (128+q) against bf16 x pairs with
// v_dot2_f32_bf16, the 128 removed through the group's sum of x.
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

constexpr int kFusedMaxPairs = 1024;

__device__ __forceinline__ void nan_row(void* Y, int y_dt, int64_t p, int64_t N, int tid, int nthreads) {
    const float nan = __uint_as_float(0x7fc00000u);
    for (int64_t j = tid; j < N; j += nthreads) store_y(Y, p * N + j, nan, y_dt);
}

// Workspace bucketing for calls with many pairs (one workgroup of 1024).
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
        if (e >= 0 && e < E)
            atomicAdd(&cnt[e], 1);
        else
            for (int64_t j = 0; j < N; j++) store_y(Y, p * N + j, __uint_as_float(0x7fc00000u), y_dt);
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
            cnt[e] = 0;  // reused as the fill cursor below
        }
        offs[U] = off;
        ws[0] = U;
    }
    __syncthreads();
    for (int64_t p = threadIdx.x; p < n_pairs; p += blockDim.x) {
        const int e = idx[p];
        if (e < 0 || e >= E) continue;
        pairs[start[e] + atomicAdd(&cnt[e], 1)] = (int)p;
    }
}

// In-block bucketing for one expert (the fused path). Returns the expert id of
// bucket u (ascending order) or -1 if fewer than u+1 experts are used; fills
// plist[0..*np) with that expert's pairs. Block-wide: every thread calls it.
__device__ int bucket_in_block(const int32_t* __restrict__ idx, int n_pairs, int E, int u,
                               int* sidx, uint32_t* pres, int* plist, int* np, int* sel,
                               void* Y, int y_dt, int64_t N) {
    const int tid = threadIdx.x, nt = blockDim.x;
    const int words = (E + 31) >> 5;
    for (int w = tid; w < words; w += nt) pres[w] = 0u;
    if (tid == 0) *np = 0;
    __syncthreads();
    for (int p = tid; p < n_pairs; p += nt) {
        const int e = idx[p];
        sidx[p] = e;
        if (e >= 0 && e < E) atomicOr(&pres[e >> 5], 1u << (e & 31));
    }
    __syncthreads();
    if (tid == 0) {
        int e_sel = -1, seen = 0;
        for (int w = 0; w < words && e_sel < 0; w++) {
            uint32_t bits = pres[w];
            const int c = __popc(bits);
            if (seen + c > u) {
                for (int k = seen; k < u; k++) bits &= bits - 1;  // drop the lower set bits
                e_sel = (w << 5) + __ffs(bits) - 1;
            }
            seen += c;
        }
        *sel = e_sel;
    }
    __syncthreads();
    const int e = *sel;
    if (e >= 0)
        for (int p = tid; p < n_pairs; p += nt)
            if (sidx[p] == e) plist[atomicAdd(np, 1)] = p;
    __syncthreads();
    return e;
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

// Rows per block = 4 waves * (64/LPR) slices * RPW rows. Weights and scales are
// read through buffer resources (rows past N read 0), so loads are
// unconditional and issue back to back; stores are predicated.
template <int LPR, int ITERS, int RPW, bool SB_F16, bool FUSED>
__global__ __launch_bounds__(256) void gather_qmv_kernel(
    const uint32_t* __restrict__ W, const uint16_t* __restrict__ S, const uint16_t* __restrict__ B,
    const uint16_t* __restrict__ X, void* __restrict__ Y, int y_dt, uint32_t N, int gs_log2,
    const int* __restrict__ ws, const int32_t* __restrict__ idx, int n_pairs, int64_t E,
    int64_t k_slots, int64_t a_vectors) {
    constexpr int SLICES = 64 / LPR;
    constexpr uint32_t P = 4 * LPR * ITERS;
    constexpr uint32_t K = 8 * P;
    __shared__ int sidx[FUSED ? kFusedMaxPairs : 1];
    __shared__ int plist_s[FUSED ? kFusedMaxPairs : 1];
    __shared__ uint32_t pres[FUSED ? kMaxExperts / 32 : 1];
    __shared__ int np_s, sel_s;
    int64_t e;
    int p_begin, p_end;
    const int* pairs;
    if constexpr (FUSED) {
        if (blockIdx.x == 0 && blockIdx.y == 0)
            for (int p = 0; p < n_pairs; p++) {
                const int ei = idx[p];
                if (ei < 0 || ei >= E) nan_row(Y, y_dt, p, N, threadIdx.x, blockDim.x);
            }
        const int es = bucket_in_block(idx, n_pairs, (int)E, blockIdx.y, sidx, pres, plist_s, &np_s,
                                       &sel_s, Y, y_dt, N);
        if (es < 0) return;  // block-uniform
        e = es;
        p_begin = 0;
        p_end = np_s;
        pairs = plist_s;
    } else {
        const int U = ws[0];
        if ((int)blockIdx.y >= U) return;
        e = ws[1 + blockIdx.y];
        p_begin = ws[1 + E + blockIdx.y];
        p_end = ws[2 + E + blockIdx.y];
        pairs = ws + 2 + 2 * E;
    }

    const int lane = threadIdx.x & 63;
    const int sl = lane % LPR, slice = lane / LPR;
    const uint32_t G = K >> gs_log2;
    const uint32_t row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * (SLICES * RPW) + slice * RPW;
    const auto rw = make_rsrc(W + e * (int64_t)N * P, N * P * 4);
    const auto rs = make_rsrc(S + e * (int64_t)N * G, N * G * 2);
    const auto rb = make_rsrc(B + e * (int64_t)N * G, N * G * 2);

    uint4 wv[RPW][ITERS];
    float sc[RPW][ITERS], bo[RPW][ITERS];
#pragma unroll
    for (int r = 0; r < RPW; r++)
#pragma unroll
        for (int it = 0; it < ITERS; it++)
            wv[r][it] = buf_load16_nt(rw, ((row0 + r) * P + it * 4 * LPR + 4 * sl) * 4);
#pragma unroll
    for (int r = 0; r < RPW; r++)
#pragma unroll
        for (int it = 0; it < ITERS; it++) {
            const uint32_t off = ((row0 + r) * G + ((32u * (it * LPR + sl)) >> gs_log2)) * 2;
            const uint16_t sh = buf_load2(rs, off), bh = buf_load2(rb, off);
            const float s = SB_F16 ? f16_to_f32(sh) : bf16_to_f32(sh);
            const float b = SB_F16 ? f16_to_f32(bh) : bf16_to_f32(bh);
            sc[r][it] = s;
            bo[r][it] = fmaf(-kCodeOffset, s, b);
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
            if (sl == LPR - 1 && row < N) {
                if (y_dt == JH_BF16)
                    static_cast<uint16_t*>(Y)[pair * N + row] = f32_to_bf16_hw(v);
                else
                    static_cast<float*>(Y)[pair * N + row] = v;
            }
        }
    }
}

template <int LPR, int ITERS, int RPW, bool SB_F16, bool FUSED>
Status run_fast_sb(const GatherArgs& a, int64_t max_u, int gs_log2, hipStream_t st) {
    constexpr int64_t rows_per_block = 4 * (64 / LPR) * RPW;
    const int64_t blocks = (a.m.rows + rows_per_block - 1) / rows_per_block;
    hipLaunchKernelGGL((gather_qmv_kernel<LPR, ITERS, RPW, SB_F16, FUSED>),
                       dim3((unsigned)blocks, (unsigned)max_u), dim3(256), 0, st, a.m.w,
                       static_cast<const uint16_t*>(a.m.scales), static_cast<const uint16_t*>(a.m.biases),
                       static_cast<const uint16_t*>(a.x), a.y, a.y_dtype, (uint32_t)a.m.rows, gs_log2,
                       static_cast<const int*>(a.workspace), a.idx, (int)(a.n_lead * a.k_slots),
                       a.n_experts, a.k_slots, a.a_vectors);
    return Status::ok();
}

template <int LPR, int ITERS, int RPW>
Status run_fast(const GatherArgs& a, int64_t max_u, int gs_log2, bool fused, hipStream_t st) {
    if (fused) {
        if (a.m.sb_dtype == JH_F16) return run_fast_sb<LPR, ITERS, RPW, true, true>(a, max_u, gs_log2, st);
        return run_fast_sb<LPR, ITERS, RPW, false, true>(a, max_u, gs_log2, st);
    }
    if (a.m.sb_dtype == JH_F16) return run_fast_sb<LPR, ITERS, RPW, true, false>(a, max_u, gs_log2, st);
    return run_fast_sb<LPR, ITERS, RPW, false, false>(a, max_u, gs_log2, st);
}

int log2_exact(int v) {
    int l = 0;
    while ((1 << l) < v) l++;
    return ((1 << l) == v) ? l : -1;
}

bool fast_tile_exists(int64_t P) {
    switch (P) {
        case 256: case 512: case 768: case 1024: case 1536: case 128: case 384:
        case 64: case 192: case 32: case 96:
            return true;
        default:
            return false;
    }
}

}  // namespace

size_t gather_workspace_bytes(int64_t n_experts, int64_t n_pairs) {
    return sizeof(int) * (size_t)(2 + 2 * n_experts + n_pairs);
}

bool gather_uses_workspace(const GatherArgs& a) {
    const int gl = log2_exact(a.m.group_size);
    const bool fast = a.x_dtype == JH_BF16 && gl >= 5 && gl <= 7 && (a.m.in % a.m.group_size) == 0 &&
                      (a.m.sb_dtype == JH_BF16 || a.m.sb_dtype == JH_F16) &&
                      (a.m.rows + 64) * (a.m.in / 2) < ((int64_t)1 << 31) && fast_tile_exists(a.m.in / 8);
    return !(fast && a.n_lead * a.k_slots <= kFusedMaxPairs);
}

Status launch_gather(const GatherArgs& a, int num_cus, hipStream_t st) {
    const int64_t n_pairs = a.n_lead * a.k_slots;
    if (n_pairs == 0) return Status::ok();
    if (a.n_experts > kMaxExperts)
        return Status::fail(JH_ERR_UNSUPPORTED, "gather_quant_matmul: more than 4096 experts");
    const int64_t max_u = n_pairs < a.n_experts ? n_pairs : a.n_experts;
    if (max_u > 65535) return Status::fail(JH_ERR_UNSUPPORTED, "gather_quant_matmul: too many experts in one call");
    const int gl = log2_exact(a.m.group_size);
    const bool fused = !gather_uses_workspace(a);
    if (!fused)
        hipLaunchKernelGGL(moe_bucket_kernel, dim3(1), dim3(1024), 0, st, a.idx, n_pairs, a.n_experts,
                           static_cast<int*>(a.workspace), a.y, a.y_dtype, a.m.rows);
    const int64_t P = a.m.in / 8;
    const bool fast_ok = a.x_dtype == JH_BF16 && gl >= 5 && gl <= 7 && (a.m.in % a.m.group_size) == 0 &&
                         (a.m.sb_dtype == JH_BF16 || a.m.sb_dtype == JH_F16) &&
                         (a.m.rows + 64) * (a.m.in / 2) < ((int64_t)1 << 31);
    if (fast_ok) {
        switch (P) {
            case 256 * 1: return run_fast<64, 1, 4>(a, max_u, gl, fused, st);
            case 256 * 2: return run_fast<64, 2, 2>(a, max_u, gl, fused, st);
            case 256 * 3: return run_fast<64, 3, 2>(a, max_u, gl, fused, st);
            case 256 * 4: return run_fast<64, 4, 1>(a, max_u, gl, fused, st);
            case 256 * 6: return run_fast<64, 6, 1>(a, max_u, gl, fused, st);
            case 128 * 1: return run_fast<32, 1, 4>(a, max_u, gl, fused, st);
            case 128 * 3: return run_fast<32, 3, 2>(a, max_u, gl, fused, st);
            case 64 * 1: return run_fast<16, 1, 4>(a, max_u, gl, fused, st);
            case 64 * 3: return run_fast<16, 3, 2>(a, max_u, gl, fused, st);
            case 32 * 1: return run_fast<8, 1, 4>(a, max_u, gl, fused, st);
            case 32 * 3: return run_fast<8, 3, 2>(a, max_u, gl, fused, st);
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
