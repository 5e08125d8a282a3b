// MoE expert products on gfx950: GatherQuantMatmul (cpu/cpu_misc.go:178-230)
// and the whole expert MLP of moeApply (qwen/moe.go:501-511).
//
// The reference buckets the (lead, slot) pairs by expert on the host and runs
// one QuantMatmul per used expert. Here the bucketing runs on the device, so the
// routing never comes back to the host, and each routed expert's packed weights
// are read once per call whatever the number of slots routed to it:
//
//  * small calls (pairs <= kInBlockMaxPairs): every block stages the
//    indices in LDS, marks the used experts in a bitmap, takes the u-th used
//    expert (ascending id, the reference's iteration order) for blockIdx.y = u
//    and collects that expert's pairs, inside the product launch;
//  * larger calls: moe_bucket_kernel writes the buckets to a workspace
//        ws[0]                  U, the number of used experts
//        ws[1 .. 1+E)           used expert ids, ascending
//        ws[1+E .. 2+2E)        bucket offsets (U+1 of them)
//        ws[2+2E .. 2+2E+pairs) pair ids (pair = lead * k_slots + slot)
//    and the product kernel reads them.
// An out-of-range index gets a row of NaN and no bucket.
//
// moe_qmv_kernel is the decode GEMV of qmv.hip (codes become bf16 128+q through
// v_perm_b32 and meet bf16 x pairs in v_dot2_f32_bf16; the 128 is removed
// through the group's sum of x) run per expert bucket: block (rb, u) loads its
// rows of expert u into registers once, then applies them to the x vector of
// every pair in the bucket. One token's slots (a single token routed to its
// top-k) skip the bucketing: block (rb, p) takes pair p's expert directly.
// Its epilogue is one of
//    EPI_PLAIN    y[pair, row]    = dot                      (GatherQuantMatmul)
//    EPI_SWIGLU   y[pair, row]    = SiLU(dot_gate) * dot_up  (two stacks, one launch)
//    EPI_PARTIAL  y[pair, row]    = score[pair] * dot        (fp32, the down product)
// The score-weighted sum over a token's slots (moeApply's Mean * K,
// qwen/moe.go:510) is taken in slot order, never by atomics, so results repeat
// bit for bit: up to 32 pairs moe_down_combine_kernel computes a token's rows
// for all its slots in one block and sums them there; beyond, EPI_PARTIAL
// products go to a workspace and moe_combine_kernel sums each token's slots.
// A whole moeApply is one SWIGLU launch over gate+up and one down launch (two
// plus the bucketing beyond 32 pairs), with h kept in bf16 between them.
#include "jh_common.hpp"

namespace jh {

__global__ __launch_bounds__(256) void qmv_generic_kernel(
    const uint32_t* __restrict__ W, const void* __restrict__ S, const void* __restrict__ B,
    int sb_dt, const void* __restrict__ X, int x_dt, void* __restrict__ Y, int y_dt, int64_t N,
    int64_t K, int gs, int bits, int64_t M, const int* __restrict__ ws, int64_t n_experts,
    int64_t k_slots, int64_t a_vectors);

namespace {

constexpr int kMaxExperts = 4096;
// Up to this many pairs every product block buckets the indices itself; beyond
// it one bucketing launch serves the call (and both products of jh_moe_swiglu):
// per-block bucketing costs each of the many blocks a dependent index load and
// four barriers (measured on MI355X at 128 pairs: gate/up 51.8 -> 40.7 us, down
// 34.8 -> 32.4 us with the buckets precomputed).
constexpr int kInBlockMaxPairs = 32;
constexpr int kMaxRouteExperts = 4096;
enum { EPI_PLAIN = 0, EPI_SWIGLU = 1, EPI_PARTIAL = 2 };
// How a product block finds its expert and pairs: the workspace buckets of
// moe_bucket_kernel, buckets made inside the block, or one pair per block.
enum { MODE_WS = 0, MODE_IN_BLOCK = 1, MODE_PAIR = 2 };
// Up to this many pairs (one token's top-8) each product block takes one pair.
constexpr int kPerPairMaxPairs = 8;

__device__ __forceinline__ void nan_row(void* Y, int y_dt, int64_t p, int64_t N, int tid, int nthreads) {
    const float nan = __uint_as_float(0x7fc00000u);
    for (int64_t j = tid; j < N; j += nthreads) store_y(Y, p * N + j, nan, y_dt);
}

// Wave-wide exclusive prefix sum (lanes in order); *total gets the sum. Every
// lane of the wave calls it.
__device__ __forceinline__ int wave_excl_scan(int v, int* total) {
    const int lane = threadIdx.x & 63;
    int s = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(s, o, 64);
        if (lane >= o) s += t;
    }
    *total = __shfl(s, 63, 64);
    return s - v;
}

// Workspace bucketing for calls with many pairs (one workgroup of 1024). Pairs
// with an out-of-range index get a NaN row in Y when Y is given. The per-expert
// offsets come from one wave's prefix sums over contiguous runs of experts.
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
        else if (Y)
            for (int64_t j = 0; j < N; j++) store_y(Y, p * N + j, __uint_as_float(0x7fc00000u), y_dt);
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        const int per = (int)((E + 63) / 64), e0 = threadIdx.x * per;
        int pairs_run = 0, used_run = 0;
        for (int j = 0; j < per; j++) {
            const int e = e0 + j;
            if (e < E) {
                pairs_run += cnt[e];
                used_run += cnt[e] > 0;
            }
        }
        int n_valid, U;
        int off = wave_excl_scan(pairs_run, &n_valid);
        int u = wave_excl_scan(used_run, &U);
        for (int j = 0; j < per; j++) {
            const int e = e0 + j;
            if (e >= E) break;
            start[e] = off;
            if (cnt[e] > 0) {
                uniq[u] = e;
                offs[u] = off;
                off += cnt[e];
                u++;
            }
            cnt[e] = 0;  // reused as the fill cursor below
        }
        if (threadIdx.x == 0) {
            ws[0] = U;
            offs[U] = n_valid;
        }
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
                               int* sidx, uint32_t* pres, int* plist, int* np, int* sel) {
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

// SiLU as the reference defines it (cpu/cpu.go:327-329): v / (1 + exp(-v)).
__device__ __forceinline__ float silu(float v) { return v / (1.0f + __expf(-v)); }

struct MoeArgs {
    const uint32_t* w[2];  // stacks [E, N, P]: [0] the only stack or gate, [1] up (SWIGLU)
    const uint16_t* s[2];  // [E, N, G] bf16 or f16
    const uint16_t* b[2];
    const uint16_t* x;     // bf16 rows of K
    void* y;               // PLAIN/SWIGLU: [pairs, N] bf16 or f32; COMBINE: f32 [n_lead, N]
    int y_dt;
    uint32_t N;            // rows per expert
    int gs_log2;
    const int* ws;         // buckets (unfused path)
    const int32_t* idx;    // [n_lead, k_slots]
    int n_pairs;
    int64_t E, k_slots, a_vectors;
    const float* scores;   // PARTIAL: [n_lead, k_slots]
};

// Expert-slot GEMV (see the file comment). LPR lanes per row, each lane ITERS
// 16-byte words per K-part; K split over KSPLIT waves that meet in LDS. Rows per
// block = (4 / KSPLIT) * (64 / LPR) * RPW.
template <int LPR, int ITERS, int RPW, int KSPLIT, bool SB_F16, int EPI, int MODE>
__global__ __launch_bounds__(256) void moe_qmv_kernel(MoeArgs a) {
    constexpr int NSTK = EPI == EPI_SWIGLU ? 2 : 1;
    constexpr int SLICES = 64 / LPR;
    constexpr int RGROUPS = 4 / KSPLIT;
    constexpr uint32_t PK = 4 * LPR * ITERS;  // words per K-part
    constexpr uint32_t P = PK * KSPLIT;
    constexpr uint32_t K = 8 * P;
    constexpr int ROWS_PER_WAVE = SLICES * RPW;
    constexpr int ROWS_PER_BLOCK = RGROUPS * ROWS_PER_WAVE;
    constexpr bool IN_BLOCK = MODE == MODE_IN_BLOCK;
    __shared__ int sidx[IN_BLOCK ? kInBlockMaxPairs : 1];
    __shared__ int plist_s[IN_BLOCK ? kInBlockMaxPairs : 1];
    __shared__ uint32_t pres[IN_BLOCK ? kMaxExperts / 32 : 1];
    __shared__ int np_s, sel_s;
    __shared__ float red[KSPLIT > 1 ? (KSPLIT - 1) * NSTK * ROWS_PER_BLOCK : 1];

    int64_t e;
    int p_begin, p_end;
    const int* pairs;
    int pair_self = 0;
    if constexpr (MODE == MODE_PAIR) {
        pair_self = blockIdx.y;
        e = a.idx[pair_self];
        if (e < 0 || e >= a.E) {  // this block's rows of the pair's output are NaN
            if (EPI != EPI_PARTIAL && blockIdx.x == 0) nan_row(a.y, a.y_dt, pair_self, a.N, threadIdx.x, blockDim.x);
            return;  // block-uniform
        }
        p_begin = 0;
        p_end = 1;
        pairs = &pair_self;
    } else if constexpr (IN_BLOCK) {
        if (EPI != EPI_PARTIAL && blockIdx.x == 0 && blockIdx.y == 0)
            for (int p = 0; p < a.n_pairs; p++) {
                const int ei = a.idx[p];
                if (ei < 0 || ei >= a.E) nan_row(a.y, a.y_dt, p, a.N, threadIdx.x, blockDim.x);
            }
        const int es = bucket_in_block(a.idx, a.n_pairs, (int)a.E, blockIdx.y, sidx, pres, plist_s,
                                       &np_s, &sel_s);
        if (es < 0) return;  // block-uniform
        e = es;
        p_begin = 0;
        p_end = np_s;
        pairs = plist_s;
    } else {
        const int U = a.ws[0];
        if ((int)blockIdx.y >= U) return;
        e = a.ws[1 + blockIdx.y];
        p_begin = a.ws[1 + a.E + blockIdx.y];
        p_end = a.ws[2 + a.E + blockIdx.y];
        pairs = a.ws + 2 + 2 * a.E;
    }

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int ks = wave % KSPLIT, rg = wave / KSPLIT;
    const int sl = lane % LPR, slice = lane / LPR;
    const uint32_t N = a.N;
    const uint32_t G = K >> a.gs_log2;
    const int slot = rg * ROWS_PER_WAVE + slice * RPW;  // first row inside the block
    const uint32_t row0 = blockIdx.x * ROWS_PER_BLOCK + slot;

    uint32_t wo[ITERS];  // word offset inside a row
#pragma unroll
    for (int it = 0; it < ITERS; it++) wo[it] = ks * PK + it * 4 * LPR + 4 * sl;

    // this block's rows of expert e, kept in registers for every pair of the bucket
    uint4 wv[NSTK][RPW][ITERS];
    float sc[NSTK][RPW][ITERS], bo[NSTK][RPW][ITERS];
#pragma unroll
    for (int t = 0; t < NSTK; t++) {
        const auto rw = make_rsrc(a.w[t] + e * (int64_t)N * P, N * P * 4);
#pragma unroll
        for (int r = 0; r < RPW; r++)
#pragma unroll
            for (int it = 0; it < ITERS; it++)
                wv[t][r][it] = buf_load16_nt(rw, ((row0 + r) * P + wo[it]) * 4);
    }
#pragma unroll
    for (int t = 0; t < NSTK; t++) {
        const auto rs = make_rsrc(a.s[t] + e * (int64_t)N * G, N * G * 2);
        const auto rb = make_rsrc(a.b[t] + e * (int64_t)N * G, N * G * 2);
#pragma unroll
        for (int r = 0; r < RPW; r++)
#pragma unroll
            for (int it = 0; it < ITERS; it++) {
                const uint32_t off = ((row0 + r) * G + ((8u * wo[it]) >> a.gs_log2)) * 2;
                const uint16_t sh = buf_load2(rs, off), bh = buf_load2(rb, off);
                const float s = SB_F16 ? f16_to_f32(sh) : bf16_to_f32(sh);
                const float b = SB_F16 ? f16_to_f32(bh) : bf16_to_f32(bh);
                sc[t][r][it] = s;
                bo[t][r][it] = fmaf(-kCodeOffset, s, b);
            }
    }

    for (int pi = p_begin; pi < p_end; pi++) {
        const int64_t pair = pairs[pi];
        const int64_t l = pair / a.k_slots, k = pair - l * a.k_slots;
        const int64_t xrow = l * a.a_vectors + (a.a_vectors == 1 ? 0 : k);
        const uint16_t* xr = a.x + xrow * K;
        float part[NSTK][RPW];
#pragma unroll
        for (int t = 0; t < NSTK; t++)
#pragma unroll
            for (int r = 0; r < RPW; r++) part[t][r] = 0.0f;
#pragma unroll
        for (int it = 0; it < ITERS; it++) {
            const uint4* xv = reinterpret_cast<const uint4*>(xr + 8 * wo[it]);
            uint32_t xp[16];
            float xs = 0.0f;
            {
                const uint4 x0 = xv[0], x1 = xv[1], x2 = xv[2], x3 = xv[3];
                xs = (pair_up(x0, &xp[0]) + pair_up(x1, &xp[4])) +
                     (pair_up(x2, &xp[8]) + pair_up(x3, &xp[12]));
            }
#pragma unroll
            for (int t = 0; t < NSTK; t++)
#pragma unroll
                for (int r = 0; r < RPW; r++) {
                    float d = 0.0f;
                    d = word_dot(wv[t][r][it].x, &xp[0], d);
                    d = word_dot(wv[t][r][it].y, &xp[4], d);
                    d = word_dot(wv[t][r][it].z, &xp[8], d);
                    d = word_dot(wv[t][r][it].w, &xp[12], d);
                    part[t][r] = fmaf(sc[t][r][it], d, part[t][r]);
                    part[t][r] = fmaf(bo[t][r][it], xs, part[t][r]);
                }
        }
#pragma unroll
        for (int t = 0; t < NSTK; t++)
#pragma unroll
            for (int r = 0; r < RPW; r++) part[t][r] = slice_sum_last<LPR>(part[t][r]);
        if constexpr (KSPLIT > 1) {
            if (ks > 0 && sl == LPR - 1)
#pragma unroll
                for (int t = 0; t < NSTK; t++)
#pragma unroll
                    for (int r = 0; r < RPW; r++)
                        red[((ks - 1) * NSTK + t) * ROWS_PER_BLOCK + slot + r] = part[t][r];
            __syncthreads();
            if (ks == 0 && sl == LPR - 1)
#pragma unroll
                for (int kp = 1; kp < KSPLIT; kp++)
#pragma unroll
                    for (int t = 0; t < NSTK; t++)
#pragma unroll
                        for (int r = 0; r < RPW; r++)
                            part[t][r] += red[((kp - 1) * NSTK + t) * ROWS_PER_BLOCK + slot + r];
            __syncthreads();  // red is rewritten by the next pair
        }
        if (ks == 0 && sl == LPR - 1) {
#pragma unroll
            for (int r = 0; r < RPW; r++) {
                const uint32_t row = row0 + r;
                if (row >= N) continue;
                if constexpr (EPI == EPI_PARTIAL) {
                    static_cast<float*>(a.y)[pair * N + row] = a.scores[pair] * part[0][r];
                } else {
                    const float v = EPI == EPI_SWIGLU ? silu(part[0][r]) * part[NSTK - 1][r] : part[0][r];
                    if (a.y_dt == JH_BF16)
                        static_cast<uint16_t*>(a.y)[pair * N + row] = f32_to_bf16_hw(v);
                    else
                        static_cast<float*>(a.y)[pair * N + row] = v;
                }
            }
        }
    }
}

__device__ __forceinline__ void store_out(void* y, int dt, int64_t i, float v) {
    if (dt == JH_BF16)
        static_cast<uint16_t*>(y)[i] = f32_to_bf16_hw(v);
    else
        static_cast<float*>(y)[i] = v;
}

// The down product and the score-weighted sum of one token's slots in one
// block (calls of up to 32 pairs): block (rb, t) has 4 waves; wave w computes
// rows rb of the experts of slots w*SPW .. w*SPW+SPW-1 against their h rows
// (all its loads issued before any is used), weights each by its score and
// adds them in slot order; the 4 waves' sums meet in LDS and are added in wave
// order. Out is written once (fp32 or bf16), so nothing clears it first, and
// the order is fixed. A token with an expert index outside [0, E) gets NaN.
// Rows per block = (64 / LPR) * RPW; K (the down's in_features) = 32 * LPR * ITERS.
// The h rows and the scores do not depend on the expert indices: they are
// requested together with the indices, ahead of the weights, so the only
// dependent round trip is index -> weights (when a lane's h chunks fit in
// registers, SPW * ITERS <= 6; longer rows load them slot by slot as before).
template <int LPR, int ITERS, int RPW, bool SB_F16, int SPW>
__global__ __launch_bounds__(256) void moe_down_combine_kernel(MoeArgs a, void* __restrict__ out, int out_dt) {
    constexpr int NW = 4;
    constexpr int SLICES = 64 / LPR;
    constexpr int ROWS = SLICES * RPW;
    constexpr uint32_t P = 4 * LPR * ITERS;
    constexpr uint32_t K = 8 * P;
    __shared__ float red[NW][ROWS];
    __shared__ int bad_s[NW];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int sl = lane % LPR, slice = lane / LPR;
    const int64_t t = blockIdx.y;
    const uint32_t N = a.N, G = K >> a.gs_log2;
    const uint32_t row0 = blockIdx.x * ROWS + slice * RPW;
    uint32_t wo[ITERS];
#pragma unroll
    for (int it = 0; it < ITERS; it++) wo[it] = it * 4 * LPR + 4 * sl;
    int64_t es[SPW];
    bool bad = false;
    int32_t eraw[SPW];
#pragma unroll
    for (int j = 0; j < SPW; j++) {
        const int64_t k = (int64_t)w * SPW + j;
        eraw[j] = k < a.k_slots ? a.idx[t * a.k_slots + k] : -1;
    }
    // the slots' h chunks and scores, in flight with the indices
    constexpr bool PRELOAD = SPW * ITERS <= 6;
    uint4 xh[PRELOAD ? SPW : 1][PRELOAD ? ITERS : 1][4];
    float score[SPW];
#pragma unroll
    for (int j = 0; j < SPW; j++) {
        const int64_t k = (int64_t)w * SPW + j;
        const int64_t pair = t * a.k_slots + (k < a.k_slots ? k : 0);
        score[j] = a.scores[pair];
        if constexpr (PRELOAD) {
            const uint16_t* xr = a.x + pair * K;
#pragma unroll
            for (int it = 0; it < ITERS; it++) {
                const uint4* xv = reinterpret_cast<const uint4*>(xr + 8 * wo[it]);
#pragma unroll
                for (int q = 0; q < 4; q++) xh[j][it][q] = xv[q];
            }
        }
    }
#pragma unroll
    for (int j = 0; j < SPW; j++) {
        const int64_t k = (int64_t)w * SPW + j;
        es[j] = -1;
        if (k < a.k_slots) {
            const int64_t e = eraw[j];
            if (e < 0 || e >= a.E) bad = true;
            else es[j] = e;
        }
    }
    // every slot's weights, scales and biases, then its h
    uint4 wv[SPW][RPW][ITERS];
    uint16_t sh[SPW][RPW][ITERS], bh[SPW][RPW][ITERS];
#pragma unroll
    for (int j = 0; j < SPW; j++) {
        const int64_t e = es[j] < 0 ? 0 : es[j];
        const auto rw = make_rsrc(a.w[0] + e * (int64_t)N * P, es[j] < 0 ? 0u : N * P * 4);
#pragma unroll
        for (int r = 0; r < RPW; r++)
#pragma unroll
            for (int it = 0; it < ITERS; it++) wv[j][r][it] = buf_load16_nt(rw, ((row0 + r) * P + wo[it]) * 4);
    }
#pragma unroll
    for (int j = 0; j < SPW; j++) {
        const int64_t e = es[j] < 0 ? 0 : es[j];
        const auto rs = make_rsrc(a.s[0] + e * (int64_t)N * G, es[j] < 0 ? 0u : N * G * 2);
        const auto rb = make_rsrc(a.b[0] + e * (int64_t)N * G, es[j] < 0 ? 0u : N * G * 2);
#pragma unroll
        for (int r = 0; r < RPW; r++)
#pragma unroll
            for (int it = 0; it < ITERS; it++) {
                const uint32_t off = ((row0 + r) * G + ((8u * wo[it]) >> a.gs_log2)) * 2;
                sh[j][r][it] = buf_load2(rs, off);
                bh[j][r][it] = buf_load2(rb, off);
            }
    }
    float acc[RPW];
#pragma unroll
    for (int r = 0; r < RPW; r++) acc[r] = 0.0f;
#pragma unroll
    for (int j = 0; j < SPW; j++) {
        const int64_t k = (int64_t)w * SPW + j;
        if (es[j] < 0) continue;  // wave-uniform
        const int64_t pair = t * a.k_slots + k;
        const uint16_t* xr = a.x + pair * K;
        float part[RPW];
#pragma unroll
        for (int r = 0; r < RPW; r++) part[r] = 0.0f;
#pragma unroll
        for (int it = 0; it < ITERS; it++) {
            uint4 x0, x1, x2, x3;
            if constexpr (PRELOAD) {
                x0 = xh[j][it][0], x1 = xh[j][it][1], x2 = xh[j][it][2], x3 = xh[j][it][3];
            } else {
                const uint4* xv = reinterpret_cast<const uint4*>(xr + 8 * wo[it]);
                x0 = xv[0], x1 = xv[1], x2 = xv[2], x3 = xv[3];
            }
            uint32_t xp[16];
            const float xs = (pair_up(x0, &xp[0]) + pair_up(x1, &xp[4])) + (pair_up(x2, &xp[8]) + pair_up(x3, &xp[12]));
#pragma unroll
            for (int r = 0; r < RPW; r++) {
                const float sc = SB_F16 ? f16_to_f32(sh[j][r][it]) : bf16_to_f32(sh[j][r][it]);
                const float bi = SB_F16 ? f16_to_f32(bh[j][r][it]) : bf16_to_f32(bh[j][r][it]);
                float d = 0.0f;
                d = word_dot(wv[j][r][it].x, &xp[0], d);
                d = word_dot(wv[j][r][it].y, &xp[4], d);
                d = word_dot(wv[j][r][it].z, &xp[8], d);
                d = word_dot(wv[j][r][it].w, &xp[12], d);
                part[r] = fmaf(sc, d, part[r]);
                part[r] = fmaf(fmaf(-kCodeOffset, sc, bi), xs, part[r]);
            }
        }
#pragma unroll
        for (int r = 0; r < RPW; r++) acc[r] += score[j] * slice_sum_last<LPR>(part[r]);
    }
    if (sl == LPR - 1)
#pragma unroll
        for (int r = 0; r < RPW; r++) red[w][slice * RPW + r] = acc[r];
    if (lane == 0) bad_s[w] = bad;
    __syncthreads();
    if (threadIdx.x < ROWS) {
        const uint32_t row = blockIdx.x * ROWS + threadIdx.x;
        if (row < N) {
            float v = ((red[0][threadIdx.x] + red[1][threadIdx.x]) + red[2][threadIdx.x]) + red[3][threadIdx.x];
            if (bad_s[0] | bad_s[1] | bad_s[2] | bad_s[3]) v = __uint_as_float(0x7fc00000u);
            store_out(out, out_dt, t * N + row, v);
        }
    }
}

// out[t, :] = the sum over slots k = 0.. of part[t * K + k, :] in slot order,
// NaN for a token with an expert index outside [0, E) (its partial rows were
// never written).
__global__ __launch_bounds__(256) void moe_combine_kernel(const float* __restrict__ part, const int32_t* __restrict__ idx,
                                                          int64_t n_tok, int64_t K, int64_t E, int64_t H,
                                                          void* __restrict__ out, int out_dt) {
    const int64_t n = n_tok * H;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t t = i / H, h = i - t * H;
        float v = 0.0f;
        bool bad = false;
        for (int64_t k = 0; k < K; k++) {
            const int32_t e = idx[t * K + k];
            if (e < 0 || e >= E) bad = true;
            else v += part[(t * K + k) * H + h];
        }
        store_out(out, out_dt, i, bad ? __uint_as_float(0x7fc00000u) : v);
    }
}

int log2_exact(int v) {
    int l = 0;
    while ((1 << l) < v) l++;
    return ((1 << l) == v) ? l : -1;
}

template <int LPR, int ITERS, int RPW, int KSPLIT, int EPI>
void run_tile(const MoeArgs& a, bool sb_f16, int mode, int64_t max_u, hipStream_t st) {
    constexpr int64_t rows_per_block = (4 / KSPLIT) * (64 / LPR) * RPW;
    const dim3 grid((unsigned)((a.N + rows_per_block - 1) / rows_per_block), (unsigned)max_u);
    auto go = [&](auto sb, auto md) {
        hipLaunchKernelGGL((moe_qmv_kernel<LPR, ITERS, RPW, KSPLIT, decltype(sb)::value, EPI, decltype(md)::value>),
                           grid, dim3(256), 0, st, a);
    };
    using T = std::true_type;
    using F = std::false_type;
    using M0 = std::integral_constant<int, MODE_WS>;
    using M1 = std::integral_constant<int, MODE_IN_BLOCK>;
    using M2 = std::integral_constant<int, MODE_PAIR>;
    if (mode == MODE_PAIR) sb_f16 ? go(T{}, M2{}) : go(F{}, M2{});
    else if (mode == MODE_IN_BLOCK) sb_f16 ? go(T{}, M1{}) : go(F{}, M1{});
    else sb_f16 ? go(T{}, M0{}) : go(F{}, M0{});
}

// Tile per row length P (32-bit words). SWIGLU holds two stacks' rows, so it
// takes half the rows per wave of the single-stack epilogues.
template <int EPI>
bool run_fast(const MoeArgs& a, int64_t P, bool sb_f16, int mode, int64_t max_u, hipStream_t st) {
    constexpr int R4 = EPI == EPI_SWIGLU ? 2 : 4;
    constexpr int R2 = EPI == EPI_SWIGLU ? 1 : 2;
    switch (P) {
        case 256 * 1: run_tile<64, 1, R4, 1, EPI>(a, sb_f16, mode, max_u, st); return true;
        case 256 * 2: run_tile<64, 2, R2, 1, EPI>(a, sb_f16, mode, max_u, st); return true;
        case 256 * 3: run_tile<64, 3, R2, 1, EPI>(a, sb_f16, mode, max_u, st); return true;
        case 256 * 4: run_tile<64, 4, 1, 1, EPI>(a, sb_f16, mode, max_u, st); return true;
        case 256 * 6: run_tile<64, 6, 1, 1, EPI>(a, sb_f16, mode, max_u, st); return true;
        case 128 * 1: run_tile<32, 1, R4, 1, EPI>(a, sb_f16, mode, max_u, st); return true;
        case 128 * 3: run_tile<32, 3, R2, 1, EPI>(a, sb_f16, mode, max_u, st); return true;
        case 64 * 1: run_tile<16, 1, R4, 1, EPI>(a, sb_f16, mode, max_u, st); return true;
        case 64 * 3: run_tile<16, 3, R2, 1, EPI>(a, sb_f16, mode, max_u, st); return true;
        case 32 * 1: run_tile<8, 1, R4, 1, EPI>(a, sb_f16, mode, max_u, st); return true;
        case 32 * 3: run_tile<8, 3, R2, 1, EPI>(a, sb_f16, mode, max_u, st); return true;
        default: return false;
    }
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

// Shapes the register-tile kernel takes: bf16 x, power-of-two groups of
// 32..128, 16-bit scales, byte offsets inside one expert below 2^31.
bool fast_ok(const QuantMatrix& m, int x_dtype) {
    const int gl = log2_exact(m.group_size);
    return m.bits == 4 && x_dtype == JH_BF16 && gl >= 5 && gl <= 7 && (m.in % m.group_size) == 0 &&
           (m.sb_dtype == JH_BF16 || m.sb_dtype == JH_F16) &&
           (m.rows + 64) * (m.in / 2) < ((int64_t)1 << 31) && fast_tile_exists(m.in / 8);
}

MoeArgs single_stack(const QuantMatrix& m) {
    MoeArgs a{};
    a.w[0] = a.w[1] = m.w;
    a.s[0] = a.s[1] = static_cast<const uint16_t*>(m.scales);
    a.b[0] = a.b[1] = static_cast<const uint16_t*>(m.biases);
    a.N = (uint32_t)m.rows;
    a.gs_log2 = log2_exact(m.group_size);
    return a;
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

}  // namespace

size_t gather_workspace_bytes(int64_t n_experts, int64_t n_pairs) {
    return sizeof(int) * (size_t)(2 + 2 * n_experts + n_pairs);
}

bool gather_uses_workspace(const GatherArgs& a) {
    return !(fast_ok(a.m, a.x_dtype) && a.n_lead * a.k_slots <= kInBlockMaxPairs);
}

Status launch_gather(const GatherArgs& a, int num_cus, hipStream_t st) {
    const int64_t n_pairs = a.n_lead * a.k_slots;
    if (n_pairs == 0) return Status::ok();
    if (a.n_experts > kMaxExperts)
        return Status::fail(JH_ERR_UNSUPPORTED, "gather_quant_matmul: more than 4096 experts");
    const int64_t max_u = n_pairs < a.n_experts ? n_pairs : a.n_experts;
    if (max_u > 65535) return Status::fail(JH_ERR_UNSUPPORTED, "gather_quant_matmul: too many experts in one call");
    const bool in_launch = !gather_uses_workspace(a);
    if (!in_launch)
        hipLaunchKernelGGL(moe_bucket_kernel, dim3(1), dim3(1024), 0, st, a.idx, n_pairs, a.n_experts,
                           static_cast<int*>(a.workspace), a.y, a.y_dtype, a.m.rows);
    const int mode = !in_launch ? MODE_WS : (n_pairs <= kPerPairMaxPairs ? MODE_PAIR : MODE_IN_BLOCK);
    if (fast_ok(a.m, a.x_dtype)) {
        MoeArgs m = single_stack(a.m);
        m.x = static_cast<const uint16_t*>(a.x);
        m.y = a.y;
        m.y_dt = a.y_dtype;
        m.ws = static_cast<const int*>(a.workspace);
        m.idx = a.idx;
        m.n_pairs = (int)n_pairs;
        m.E = a.n_experts;
        m.k_slots = a.k_slots;
        m.a_vectors = a.a_vectors;
        if (run_fast<EPI_PLAIN>(m, a.m.in / 8, a.m.sb_dtype == JH_F16, mode, mode == MODE_PAIR ? n_pairs : max_u,
                                st))
            return Status::ok();
    }
    int64_t blocks = (a.m.rows + 3) / 4;
    const int64_t cap = (int64_t)num_cus * 4;
    if (blocks > cap) blocks = cap;
    hipLaunchKernelGGL(qmv_generic_kernel, dim3((unsigned)blocks, (unsigned)max_u), dim3(256), 0, st,
                       a.m.w, a.m.scales, a.m.biases, a.m.sb_dtype, a.x, a.x_dtype, a.y, a.y_dtype,
                       a.m.rows, a.m.in, a.m.group_size, a.m.bits, (int64_t)0,
                       static_cast<const int*>(a.workspace), a.n_experts, a.k_slots, a.a_vectors);
    return Status::ok();
}

// ---- router: softmax over the experts, top-k, optional renormalisation ----------
//
// One wave per token, the arithmetic of the CPU backend step by step so that the
// chosen experts and their scores are bit-identical to it: the row max; e_i =
// fl32(exp(fl64(fl32(v_i - max)))) (cpu/cpu.go:461-499); the sum of the e_i in
// index order by one lane; p_i = e_i / sum. Top-k is the reference's selection
// sort (qwen/moe.go:420-444): pass i takes the first position j >= i (in the
// current order array) holding the largest probability, then swaps order[i] and
// order[j]. Each pass is a wave-wide argmax with ties going to the smaller j,
// which is the strict '>' scan. Renormalisation divides by the in-order sum of
// the k scores when it is positive (qwen/moe.go:472-481).
__global__ __launch_bounds__(64) void moe_route_kernel(const void* __restrict__ logits, int l_dt, int E, int k,
                                                       int norm, int32_t* __restrict__ idx_out,
                                                       float* __restrict__ score_out) {
    __shared__ float p[kMaxRouteExperts];
    __shared__ int order[kMaxRouteExperts];
    __shared__ float sum_s;
    const int lane = threadIdx.x;
    const int64_t t = blockIdx.x;
    float mx = -__builtin_inff();
    for (int i = lane; i < E; i += 64) {
        const float v = l_dt == JH_BF16 ? bf16_to_f32(static_cast<const uint16_t*>(logits)[t * E + i])
                                        : static_cast<const float*>(logits)[t * E + i];
        p[i] = v;
        order[i] = i;
        mx = fmaxf(mx, v);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    for (int i = lane; i < E; i += 64) p[i] = (float)exp((double)(p[i] - mx));
    __syncthreads();
    if (lane == 0) {
        float s = 0.0f;
        for (int i = 0; i < E; i++) s += p[i];
        sum_s = s;
    }
    __syncthreads();
    const float sum = sum_s;
    for (int i = lane; i < E; i += 64) p[i] = p[i] / sum;
    __syncthreads();
    for (int it = 0; it < k; it++) {
        float bv = -__builtin_inff();
        int bj = E;
        for (int j = it + lane; j < E; j += 64) {
            const float v = p[order[j]];
            if (v > bv) bv = v, bj = j;
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const int oj = __shfl_xor(bj, o, 64);
            if (ov > bv || (ov == bv && oj < bj)) bv = ov, bj = oj;
        }
        if (lane == 0 && bj < E) {
            const int a = order[it];
            order[it] = order[bj];
            order[bj] = a;
        }
        __syncthreads();
    }
    if (lane == 0) {
        float s = 0.0f;
        for (int i = 0; i < k; i++) s += p[order[i]];
        sum_s = s;
    }
    __syncthreads();
    const float ks = sum_s;
    for (int i = lane; i < k; i += 64) {
        float v = p[order[i]];
        if (norm && ks > 0.0f) v = v / ks;
        idx_out[t * k + i] = order[i];
        score_out[t * k + i] = v;
    }
}

Status launch_moe_route(const void* logits, int l_dt, int64_t n_tok, int E, int k, bool norm, int32_t* idx,
                        float* scores, hipStream_t st) {
    if (n_tok == 0 || k == 0) return Status::ok();
    if (E > kMaxRouteExperts) return Status::fail(JH_ERR_UNSUPPORTED, "moe_route: more than 4096 experts");
    if (n_tok > 0x7fffffff) return Status::fail(JH_ERR_UNSUPPORTED, "moe_route: too many tokens");
    hipLaunchKernelGGL(moe_route_kernel, dim3((unsigned)n_tok), dim3(64), 0, st, logits, l_dt, E, k, norm ? 1 : 0,
                       idx, scores);
    return Status::ok();
}

const char* moe_unsupported(const MoeMlpArgs& a) {
    if (a.n_experts > kMaxExperts) return "more than 4096 experts";
    if (a.gate.rows != a.up.rows || a.gate.in != a.up.in || a.down.in != a.gate.rows)
        return "gate/up must be [E, I, H] and down [E, H, I]";
    if (a.gate.sb_dtype != a.up.sb_dtype || a.gate.sb_dtype != a.down.sb_dtype)
        return "the three stacks must share one scale dtype";
    if (!fast_ok(a.gate, JH_BF16) || !fast_ok(a.down, JH_BF16))
        return "shape outside the expert tiles (bf16 scales, group 32/64/128, H and I in "
               "{256, 512, 768, 1024, 1536, 2048, 3072, 4096, 6144, 8192, 12288})";
    const int64_t max_u = std::min<int64_t>(a.n_tok * a.k_slots, a.n_experts);
    if (max_u > 65535) return "too many experts in one call";
    return nullptr;
}

// The calls whose down product and combine run as one launch per token
// (moe_down_combine_kernel): up to 32 pairs and 16 slots per token.
bool moe_small(const MoeMlpArgs& a) {
    return a.n_tok * a.k_slots <= kInBlockMaxPairs && a.k_slots <= 16;
}

template <int LPR, int ITERS, int SPW>
void run_down_combine(const MoeArgs& d, bool f16, int64_t n_tok, void* out, int out_dt, hipStream_t st) {
    constexpr int rows = 64 / LPR;
    const dim3 grid((unsigned)((d.N + rows - 1) / rows), (unsigned)n_tok);
    if (f16)
        hipLaunchKernelGGL((moe_down_combine_kernel<LPR, ITERS, 1, true, SPW>), grid, dim3(256), 0, st, d, out, out_dt);
    else
        hipLaunchKernelGGL((moe_down_combine_kernel<LPR, ITERS, 1, false, SPW>), grid, dim3(256), 0, st, d, out, out_dt);
}

template <int SPW>
bool down_combine_tiles(const MoeArgs& d, int64_t P, bool f16, int64_t n_tok, void* out, int out_dt, hipStream_t st) {
    switch (P) {
        case 256 * 1: run_down_combine<64, 1, SPW>(d, f16, n_tok, out, out_dt, st); return true;
        case 256 * 2: run_down_combine<64, 2, SPW>(d, f16, n_tok, out, out_dt, st); return true;
        case 256 * 3: run_down_combine<64, 3, SPW>(d, f16, n_tok, out, out_dt, st); return true;
        case 256 * 4: run_down_combine<64, 4, SPW>(d, f16, n_tok, out, out_dt, st); return true;
        case 256 * 6: run_down_combine<64, 6, SPW>(d, f16, n_tok, out, out_dt, st); return true;
        case 128 * 1: run_down_combine<32, 1, SPW>(d, f16, n_tok, out, out_dt, st); return true;
        case 128 * 3: run_down_combine<32, 3, SPW>(d, f16, n_tok, out, out_dt, st); return true;
        case 64 * 1: run_down_combine<16, 1, SPW>(d, f16, n_tok, out, out_dt, st); return true;
        case 64 * 3: run_down_combine<16, 3, SPW>(d, f16, n_tok, out, out_dt, st); return true;
        case 32 * 1: run_down_combine<8, 1, SPW>(d, f16, n_tok, out, out_dt, st); return true;
        case 32 * 3: run_down_combine<8, 3, SPW>(d, f16, n_tok, out, out_dt, st); return true;
        default: return false;
    }
}

size_t moe_workspace_bytes(const MoeMlpArgs& a) {
    const int64_t n_pairs = a.n_tok * a.k_slots;
    size_t b = align256(sizeof(uint16_t) * (size_t)(n_pairs * a.gate.rows));  // h
    if (!moe_small(a)) {
        b += align256(sizeof(float) * (size_t)(n_pairs * a.down.rows));  // weighted down partials
        b += gather_workspace_bytes(a.n_experts, n_pairs);
    }
    return b;
}

Status launch_moe_mlp(const MoeMlpArgs& a, void* workspace, hipStream_t st) {
    const int64_t n_pairs = a.n_tok * a.k_slots;
    if (a.n_tok == 0) return Status::ok();
    if (const char* why = moe_unsupported(a)) return Status::fail(JH_ERR_UNSUPPORTED, std::string("moe_swiglu: ") + why);
    const int64_t H = a.down.rows, I = a.gate.rows;
    const int64_t max_u = std::min<int64_t>(n_pairs, a.n_experts);
    const bool small = moe_small(a);
    const bool f16 = a.gate.sb_dtype == JH_F16;
    char* wsp = static_cast<char*>(workspace);
    uint16_t* h = reinterpret_cast<uint16_t*>(wsp);
    wsp += align256(sizeof(uint16_t) * (size_t)(n_pairs * I));
    float* part = nullptr;
    int* buckets = nullptr;
    if (!small) {
        part = reinterpret_cast<float*>(wsp);
        wsp += align256(sizeof(float) * (size_t)(n_pairs * H));
        buckets = reinterpret_cast<int*>(wsp);
    }
    const int64_t n_out = a.n_tok * H;
    const unsigned out_blocks = (unsigned)std::min<int64_t>((n_out + 255) / 256, 4096);
    if (n_pairs == 0) {  // every token's sum is empty
        hipLaunchKernelGGL(moe_combine_kernel, dim3(out_blocks), dim3(256), 0, st, static_cast<const float*>(nullptr),
                           a.idx, a.n_tok, (int64_t)0, a.n_experts, H, a.out, a.out_dtype);
        return Status::ok();
    }
    if (!small)
        hipLaunchKernelGGL(moe_bucket_kernel, dim3(1), dim3(1024), 0, st, a.idx, n_pairs, a.n_experts, buckets,
                           static_cast<void*>(nullptr), (int)JH_BF16, (int64_t)0);
    const int gu_mode = !small ? MODE_WS : (n_pairs <= kPerPairMaxPairs ? MODE_PAIR : MODE_IN_BLOCK);

    MoeArgs g = single_stack(a.gate);
    g.w[1] = a.up.w;
    g.s[1] = static_cast<const uint16_t*>(a.up.scales);
    g.b[1] = static_cast<const uint16_t*>(a.up.biases);
    g.x = static_cast<const uint16_t*>(a.x);
    g.y = h;
    g.y_dt = JH_BF16;
    g.ws = buckets;
    g.idx = a.idx;
    g.n_pairs = (int)n_pairs;
    g.E = a.n_experts;
    g.k_slots = a.k_slots;
    g.a_vectors = 1;
    if (!run_fast<EPI_SWIGLU>(g, a.gate.in / 8, f16, gu_mode, gu_mode == MODE_PAIR ? n_pairs : max_u, st))
        return Status::fail(JH_ERR_UNSUPPORTED, "moe_swiglu: no tile for the gate/up shape");

    MoeArgs d = single_stack(a.down);
    d.x = h;
    d.ws = buckets;
    d.idx = a.idx;
    d.n_pairs = (int)n_pairs;
    d.E = a.n_experts;
    d.k_slots = a.k_slots;
    d.a_vectors = a.k_slots;
    d.scores = a.scores;
    const int64_t Pd = a.down.in / 8;
    if (small) {
        const bool ok = a.k_slots <= 4   ? down_combine_tiles<1>(d, Pd, f16, a.n_tok, a.out, a.out_dtype, st)
                        : a.k_slots <= 8 ? down_combine_tiles<2>(d, Pd, f16, a.n_tok, a.out, a.out_dtype, st)
                                         : down_combine_tiles<4>(d, Pd, f16, a.n_tok, a.out, a.out_dtype, st);
        if (!ok) return Status::fail(JH_ERR_UNSUPPORTED, "moe_swiglu: no tile for the down shape");
        return Status::ok();
    }
    d.y = part;
    d.y_dt = JH_F32;
    if (!run_fast<EPI_PARTIAL>(d, Pd, f16, MODE_WS, max_u, st))
        return Status::fail(JH_ERR_UNSUPPORTED, "moe_swiglu: no tile for the down shape");
    hipLaunchKernelGGL(moe_combine_kernel, dim3(out_blocks), dim3(256), 0, st, static_cast<const float*>(part),
                       a.idx, a.n_tok, a.k_slots, a.n_experts, H, a.out, a.out_dtype);
    return Status::ok();
}

}  // namespace jh
