// The decode GEMV tile for MLX affine 4- and 8-bit weights on gfx950, shared by
// the plain product kernels (qmv.hip) and the fused q/k/v product + attention
// launch (decode.hip). The design notes are at the top of qmv.hip.
#pragma once

#include "jh_common.hpp"

namespace jh {
namespace qmvt {

// The slice sums of RPW values at once: each DPP step is applied to all RPW
// values before the next, so the DPP read-after-write waits are filled with
// useful work. Totals land in the last lane of each slice (see slice_sum_last).
template <int LPR, int RPW>
__device__ __forceinline__ void slice_sums_last(float (&v)[RPW]) {
    auto step = [&](auto ctrl, auto row_mask) {
#pragma unroll
        for (int r = 0; r < RPW; r++)
            v[r] += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                                  0, __builtin_bit_cast(int, v[r]), decltype(ctrl)::value,
                                                  decltype(row_mask)::value, 0xF, false));
    };
    using All = std::integral_constant<int, 0xF>;
    if constexpr (LPR >= 2) step(std::integral_constant<int, 0x111>{}, All{});
    if constexpr (LPR >= 4) step(std::integral_constant<int, 0x112>{}, All{});
    if constexpr (LPR >= 8) step(std::integral_constant<int, 0x114>{}, All{});
    if constexpr (LPR >= 16) step(std::integral_constant<int, 0x118>{}, All{});
    if constexpr (LPR >= 32) step(std::integral_constant<int, 0x142>{}, std::integral_constant<int, 0xA>{});
    if constexpr (LPR >= 64) step(std::integral_constant<int, 0x143>{}, std::integral_constant<int, 0xC>{});
}

// Stores RPW consecutive outputs from one lane (vector store when all are in
// range and RPW is 2 or 4).
template <int RPW>
__device__ __forceinline__ void store_rows(void* Y, int y_dt, uint32_t row0, uint32_t N,
                                           const float (&v)[RPW]) {
    if constexpr (RPW == 2 || RPW == 4) {
        if (row0 + RPW <= N) {
            if (y_dt == JH_BF16) {
                uint32_t pk[RPW / 2];
#pragma unroll
                for (int r = 0; r < RPW; r += 2)
                    pk[r / 2] = (uint32_t)f32_to_bf16_hw(v[r]) | ((uint32_t)f32_to_bf16_hw(v[r + 1]) << 16);
                if constexpr (RPW == 4)
                    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(Y) + row0) = make_uint2(pk[0], pk[1]);
                else
                    *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(Y) + row0) = pk[0];
            } else {
                float* yf = static_cast<float*>(Y) + row0;
                if constexpr (RPW == 4)
                    *reinterpret_cast<float4*>(yf) = make_float4(v[0], v[1], v[2], v[3]);
                else
                    *reinterpret_cast<float2*>(yf) = make_float2(v[0], v[1]);
            }
            return;
        }
    }
#pragma unroll
    for (int r = 0; r < RPW; r++)
        if (row0 + r < N) {
            if (y_dt == JH_BF16)
                static_cast<uint16_t*>(Y)[row0 + r] = f32_to_bf16_hw(v[r]);
            else
                static_cast<float*>(Y)[row0 + r] = v[r];
        }
}

// Decode GEMV tile:
//   LPR    lanes per row slice (64 / LPR row slices per wave)
//   ITERS  16-byte weight loads per lane per row and K part
//   RPW    consecutive rows per slice per pass
//   KSPLIT waves sharing one row (each takes 1/KSPLIT of K); their partial sums
//          meet in LDS. A block has 4 waves = 4 / KSPLIT row groups.
// Words per row P = 4 * LPR * ITERS * KSPLIT (K = 32 * LPR * ITERS * KSPLIT).
// The grid strides over passes of whole blocks (block-uniform loop, so the
// LDS barriers are reached by all waves). Weights and scales are read through
// buffer resources: rows past N read as zero, so every load is unconditional
// and issues back to back; only the stores are predicated.
// Fusions around the product (decode only), chosen at compile time:
//   PRO_NONE     x is bf16 [K]
//   PRO_RMSNORM  x is the fp32 residual stream [K]; y = RMSNorm(x, nw) . W^T
//                (cpu/cpu_ops.go:144-162) as (bf16(x * nw) . W^T) / sqrt(mean(x^2)
//                + eps): the product is linear in its input, so the 1/rms factor
//                is applied to the fp32 dot products and nothing waits for the
//                sum of squares before them. Each wave sums x^2 over its K part;
//                the parts meet in LDS at the first pass's K-split exchange.
//   EPI_STORE    y = dot
//   EPI_RESID    y (fp32) = resid + dot; resid may alias y (the residual Add of
//                qwen/block.go:59-60 done in place).
//   EPI_SWIGLU   W holds 2N rows, the gate rows then the up rows; y[j] =
//                SiLU(dot_j) * dot_{N+j} (MLP.Forward's Mul(SiLU(gate), up),
//                qwen/mlp.go:33-35). A slice computes RPW/2 gate rows and the
//                matching up rows, so both dots meet in one lane.
//   PRO_NORMED   x is bf16(h * nw) from an EPI_RESID_NORM product, with the
//                sum of h^2 in kNormSlots partials: each wave sums its share of
//                the partials (loaded ahead of the weights), and the epilogue
//                scales as PRO_RMSNORM does, so x costs what a plain one does.
//   PRO_XF32     x is fp32 [K] (the activation type of the CPU backend and of
//                Dequantize), rounded to bf16 (nearest even) and then used as
//                PRO_NONE uses its x, so the result has the bits of a bf16-x
//                call on bf16(x). A lane's 32-element run is 128 bytes of fp32:
//                read lane by lane that is 8 loads with a 128-byte lane stride
//                (4x the cache lines of the bf16 loads). Instead each wave reads
//                its K part with consecutive lanes on consecutive 16 bytes,
//                rounds it to bf16 into LDS, and every lane takes its run from
//                there, as it would from a bf16 x.
//   EPI_RESID_NORM  EPI_RESID, plus the next norm's input: nout[row] =
//                bf16(y * nw[row]) and, per block, the sum of y^2 over its rows
//                in stats[blockIdx.x] (grid <= kNormSlots; block 0 zeroes the
//                unused slots). Fixed order: deterministic.
enum { PRO_NONE = 0, PRO_RMSNORM = 1, PRO_NORMED = 3, PRO_XF32 = 4 };
constexpr int kProSiluMul = 2;  // x = [gate | up]: composed from separate launches
enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2, EPI_RESID_NORM = 3 };

struct QmvFusion {
    const uint16_t* nw = nullptr;  // bf16 norm weight: [K] (PRO_RMSNORM) or [N] (EPI_RESID_NORM)
    float eps = 0.0f;
    const float* resid = nullptr;  // fp32 [N] (EPI_RESID, EPI_RESID_NORM)
    float* stats = nullptr;        // kNormSlots (PRO_NORMED: in; EPI_RESID_NORM: out)
    uint16_t* nout = nullptr;      // bf16 [N] (EPI_RESID_NORM)
};

// Rows of one block pass: 4 waves = 4 / KSPLIT row groups of 64 / LPR slices.
template <int LPR, int RPW, int KSPLIT, int EPI>
constexpr uint32_t qmv_rows_per_block() {
    return (4 / KSPLIT) * (64 / LPR) * (EPI == EPI_SWIGLU ? RPW / 2 : RPW);
}

// Block passes over consecutive rows (the plain product).
struct LinearRows {
    uint32_t rpb;
    __device__ uint32_t base(uint32_t blk) const { return blk * rpb; }
};

// The tile's work for one block: logical block passes blk0, blk0 + bstride, ...
// below nblk, pass blk covering output rows rmap.base(blk) .. + rows per block
// (a base at or past N reads zero weights and stores nothing).
template <int LPR, int ITERS, int RPW, int KSPLIT, bool SB_F16, int PRO = PRO_NONE, int EPI = EPI_STORE,
          int BITS = 4, bool PIPE = false, class RowMap = LinearRows>
__device__ __forceinline__ void qmv_tile(
    const uint32_t* __restrict__ W, const uint16_t* __restrict__ S,
    const uint16_t* __restrict__ B, const void* __restrict__ Xv, void* Y,
    int y_dt, uint32_t N, int gs_log2, const QmvFusion& fu, uint32_t blk0, uint32_t bstride, uint32_t nblk,
    RowMap rmap) {
    constexpr int SLICES = 64 / LPR;
    constexpr int RGROUPS = 4 / KSPLIT;                 // row groups per block
    constexpr uint32_t PK = 4 * LPR * ITERS;            // words per K part
    constexpr uint32_t P = PK * KSPLIT;
    constexpr int RO = EPI == EPI_SWIGLU ? RPW / 2 : RPW;  // output rows per slice and pass
    constexpr int ROWS_PER_WAVE = SLICES * RO;
    static_assert(RGROUPS * ROWS_PER_WAVE == (int)qmv_rows_per_block<LPR, RPW, KSPLIT, EPI>(), "rows per block");
    static_assert(EPI != EPI_SWIGLU || RPW % 2 == 0, "SwiGLU pairs gate and up rows");
    static_assert(BITS == 4 || (BITS == 8 && PRO != PRO_RMSNORM), "8-bit tiles take a bf16 x");
    // 8-bit codes are read as two 4-bit halves, q = lo + 16 hi, against a virtual
    // input that holds each x twice: (x, 16x) for the (lo, hi) nibbles of its
    // byte. 16x is exact in bf16, so the word dots are the 4-bit ones, and the
    // offset 128 of each nibble sums to 128 * 17 per element.
    constexpr uint32_t EPW = 32 / BITS;                 // elements per word
    constexpr float OFF = BITS == 4 ? kCodeOffset : 17.0f * kCodeOffset;
    const uint32_t NW = EPI == EPI_SWIGLU ? 2 * N : N;     // rows of W
    const int lane = threadIdx.x & 63;
    const int wv_id = threadIdx.x >> 6;
    const int ks = wv_id % KSPLIT, rg = wv_id / KSPLIT;
    const int sl = lane % LPR;
    const int slice = lane / LPR;
    const uint32_t G = (P * EPW) >> gs_log2;  // groups per row
    const auto rw = make_rsrc(W, NW * P * 4);
    const auto rs = make_rsrc(S, NW * G * 2);
    const auto rb = make_rsrc(B, NW * G * 2);
    __shared__ float red[(KSPLIT > 1) ? (KSPLIT - 1) * RGROUPS * SLICES * RPW : 1];
    __shared__ float ssq[4];
    constexpr uint32_t K = EPW * P;

    uint32_t gi[ITERS], wo[ITERS];
#pragma unroll
    for (int it = 0; it < ITERS; it++) {
        wo[it] = ks * PK + it * 4 * LPR + 4 * sl;   // word offset inside a row
        gi[it] = (EPW * wo[it]) >> gs_log2;
    }
    // PIPE: two register sets; the next pass's loads are issued before this
    // pass is computed (a persistent grid of a few blocks per CU walks the rows)
    constexpr int NB = PIPE ? 2 : 1;
    uint4 wv[NB][RPW][ITERS];
    uint16_t sh[NB][RPW][ITERS], bh[NB][RPW][ITERS];
    constexpr bool RESID = EPI == EPI_RESID || EPI == EPI_RESID_NORM;
    float rv[NB][RESID ? RPW : 1];  // the residual rows, fetched with the pass's weights
    uint16_t nv[NB][EPI == EPI_RESID_NORM ? RPW : 1];  // the next norm's weights for those rows
    const auto rr = make_rsrc(fu.resid, RESID ? N * 4 : 0);
    const auto rn = make_rsrc(fu.nw, EPI == EPI_RESID_NORM ? N * 2 : 0);
    // Loads complete in issue order. The raw x loads go first, then the first
    // pass's weights (which do not depend on x), and only then is x regrouped:
    // that waits for x alone while the weights are still in flight. Rows past the
    // matrix read as zero (buffer bounds).
    auto wrow = [&](uint32_t row0, int r) -> uint32_t {
        return EPI == EPI_SWIGLU ? row0 + (r % RO) + (r / RO) * N : row0 + r;
    };
    // Row by row: a row's words, then its scales and biases, so that the first
    // rows' dot products can start while later rows are still arriving (loads
    // complete in issue order).
    auto load_pass = [&](auto bufc, uint32_t row0) {
        constexpr int Q = decltype(bufc)::value;
#pragma unroll
        for (int r = 0; r < RPW; r++) {
#pragma unroll
            for (int it = 0; it < ITERS; it++)
                wv[Q][r][it] = buf_load16_nt(rw, (wrow(row0, r) * P + wo[it]) * 4);
#pragma unroll
            for (int it = 0; it < ITERS; it++) {
                const uint32_t off = (wrow(row0, r) * G + gi[it]) * 2;
                sh[Q][r][it] = buf_load2(rs, off);
                bh[Q][r][it] = buf_load2(rb, off);
            }
        }
        if constexpr (RESID)
#pragma unroll
            for (int r = 0; r < RPW; r++)
                rv[Q][r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rr, (row0 + r) * 4, 0, 0));
        if constexpr (EPI == EPI_RESID_NORM)
#pragma unroll
            for (int r = 0; r < RPW; r++) nv[Q][r] = buf_load2(rn, (row0 + r) * 2);
    };
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, NB - 1>;
    // raw x: 32 (4-bit) or 16 (8-bit) elements per lane per ITER (bf16, or fp32
    // for the norm)
    constexpr int XW = PRO == PRO_RMSNORM ? 8 : (int)EPW / 2;  // 16-byte chunks of them
    uint4 xraw[ITERS][XW];
    uint4 xaux[ITERS][4];  // norm weights (PRO_RMSNORM)
    // PRO_XF32: the wave's K part of x (EPW * PK elements) in 16-byte chunks,
    // chunk c read by lane c % 64, and its bf16 copy in LDS (one region per wave)
    constexpr uint32_t XE = EPW * PK;                            // fp32 elements of a wave's K part
    constexpr int XC = PRO == PRO_XF32 ? (int)((XE / 4 + 63) / 64) : 1;  // chunks per lane
    uint4 xf32[XC];
    __shared__ uint2 xstage[PRO == PRO_XF32 ? 4 * (XE / 4) : 1];  // 4 waves x XE bf16
    if constexpr (PRO == PRO_XF32) {
        const auto rxf = make_rsrc(static_cast<const float*>(Xv) + ks * XE, XE * 4);
#pragma unroll
        for (int c = 0; c < XC; c++) {
            const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rxf, (uint32_t)(c * 64 + lane) * 16, 0, 0);
            xf32[c] = make_uint4(v.x, v.y, v.z, v.w);
        }
    }
#pragma unroll
    for (int it = 0; it < ITERS; it++) {
        const uint32_t e0 = EPW * wo[it];
        if constexpr (PRO == PRO_RMSNORM) {
            const uint4* xv = reinterpret_cast<const uint4*>(static_cast<const float*>(Xv) + e0);
#pragma unroll
            for (int j = 0; j < 8; j++) xraw[it][j] = xv[j];
        } else if constexpr (PRO == PRO_XF32) {
            // taken from LDS after the weights are requested
        } else {
            const uint4* xv = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(Xv) + e0);
#pragma unroll
            for (int j = 0; j < XW; j++) xraw[it][j] = xv[j];
        }
    }
    // the norm weights go with x, ahead of the weights, so the normalisation
    // waits for x and them alone
    if constexpr (PRO == PRO_RMSNORM) {
#pragma unroll
        for (int it = 0; it < ITERS; it++) {
            const uint4* av = reinterpret_cast<const uint4*>(fu.nw + 8u * wo[it]);
#pragma unroll
            for (int j = 0; j < 4; j++) xaux[it][j] = av[j];
        }
    }
    // PRO_NORMED: this wave's share of the statistics partials, ahead of the weights
    constexpr int SPL = PRO == PRO_NORMED ? kNormSlots / KSPLIT / 256 : 1;  // float4 per lane
    static_assert(PRO != PRO_NORMED || SPL >= 1, "statistics split");
    float4 st4[SPL];
    if constexpr (PRO == PRO_NORMED) {
        const float4* sp = reinterpret_cast<const float4*>(fu.stats) + ks * (kNormSlots / KSPLIT / 4);
#pragma unroll
        for (int j = 0; j < SPL; j++) st4[j] = sp[j * 64 + lane];
    }
    const uint32_t lane_row = rg * ROWS_PER_WAVE + (uint32_t)slice * RO;
    load_pass(B0{}, rmap.base(blk0) + lane_row);
    // the product's input as bf16, 8 per uint4
    uint4 xin[ITERS][4];
    float ss_part = 0.0f;  // PRO_RMSNORM / PRO_NORMED: sum of x^2 over this wave's share
    float sq = 0.0f;       // EPI_RESID_NORM: sum of y^2 over the rows this lane stores
    if constexpr (PRO == PRO_NORMED) {
        float t = 0.0f;
#pragma unroll
        for (int j = 0; j < SPL; j++) t += (st4[j].x + st4[j].y) + (st4[j].z + st4[j].w);
        ss_part = wave_sum(t);  // every lane holds the wave's share
        if constexpr (KSPLIT > 1)
            if (lane == 0) ssq[wv_id] = ss_part;
    }
    if constexpr (PRO == PRO_XF32) {
        // fp32 chunks to bf16 (nearest even) in the wave's LDS region, then each
        // lane's runs in the layout a bf16 x loads as
        auto cvt2 = [](uint32_t a, uint32_t b) {
            return (uint32_t)f32_to_bf16_hw(__uint_as_float(a)) | ((uint32_t)f32_to_bf16_hw(__uint_as_float(b)) << 16);
        };
        uint2* xw = xstage + wv_id * (XE / 4);
#pragma unroll
        for (int c = 0; c < XC; c++)
            if ((uint32_t)(c * 64 + lane) < XE / 4)
                xw[c * 64 + lane] = make_uint2(cvt2(xf32[c].x, xf32[c].y), cvt2(xf32[c].z, xf32[c].w));
        __syncthreads();
#pragma unroll
        for (int it = 0; it < ITERS; it++) {
            const uint4* src = reinterpret_cast<const uint4*>(xw + (EPW * (wo[it] - ks * PK)) / 4);
#pragma unroll
            for (int j = 0; j < XW; j++) xraw[it][j] = src[j];
        }
    }
    float xs8[ITERS];  // 8-bit: the sum of the real inputs
    if constexpr (BITS == 8) {
        // word j of a 16-byte chunk holds elements 4j..4j+3: its virtual input is
        // (x, 16x) per element, 8 bf16 in one uint4
#pragma unroll
        for (int it = 0; it < ITERS; it++) {
            const uint32_t xr[8] = {xraw[it][0].x, xraw[it][0].y, xraw[it][0].z, xraw[it][0].w,
                                    xraw[it][1].x, xraw[it][1].y, xraw[it][1].z, xraw[it][1].w};
            float sum = 0.0f;
            uint32_t v[16];
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const float a = __uint_as_float(xr[q] << 16), b = __uint_as_float(xr[q] & 0xFFFF0000u);
                sum += a + b;
                v[2 * q] = (xr[q] & 0xFFFFu) | ((uint32_t)f32_to_bf16_hw(16.0f * a) << 16);
                v[2 * q + 1] = (xr[q] >> 16) | ((uint32_t)f32_to_bf16_hw(16.0f * b) << 16);
            }
#pragma unroll
            for (int j = 0; j < 4; j++) xin[it][j] = make_uint4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
            xs8[it] = sum;
        }
    } else if constexpr (PRO == PRO_NONE || PRO == PRO_NORMED || PRO == PRO_XF32) {
#pragma unroll
        for (int it = 0; it < ITERS; it++)
#pragma unroll
            for (int j = 0; j < 4; j++) xin[it][j] = xraw[it][j];
    } else {
        // x * nw to bf16, and the sum of squares of this wave's K part (each
        // slice holds the whole part)
        float ss = 0.0f;
#pragma unroll
        for (int it = 0; it < ITERS; it++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint4 a = xraw[it][2 * j], b = xraw[it][2 * j + 1], w = xaux[it][j];
                const float xs8[8] = {__uint_as_float(a.x), __uint_as_float(a.y), __uint_as_float(a.z),
                                      __uint_as_float(a.w), __uint_as_float(b.x), __uint_as_float(b.y),
                                      __uint_as_float(b.z), __uint_as_float(b.w)};
                const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
                uint32_t o[4];
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    ss = fmaf(xs8[2 * q], xs8[2 * q], ss);
                    ss = fmaf(xs8[2 * q + 1], xs8[2 * q + 1], ss);
                    const float n0 = xs8[2 * q] * __uint_as_float(ww[q] << 16);
                    const float n1 = xs8[2 * q + 1] * __uint_as_float(ww[q] & 0xFFFF0000u);
                    o[q] = (uint32_t)f32_to_bf16_hw(n0) | ((uint32_t)f32_to_bf16_hw(n1) << 16);
                }
                xin[it][j] = make_uint4(o[0], o[1], o[2], o[3]);
            }
        ss_part = slice_sum_last<LPR>(ss);  // valid in the slice's last lane
        if constexpr (KSPLIT > 1)
            if (slice == 0 && sl == LPR - 1) ssq[wv_id] = ss_part;
    }

    // this lane's part of x, as (x_p, x_{p+4}) bf16 pairs, and its sums
    uint32_t xp[ITERS][16];
    float xs[ITERS];
#pragma unroll
    for (int it = 0; it < ITERS; it++) {
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) sum += pair_up(xin[it][j], &xp[it][4 * j]);
        xs[it] = BITS == 8 ? xs8[it] : sum;
    }
    // every row's dot product starts from -OFF * sum(x), so the codes' offset
    // cancels inside it and a row's group term is scale * dot + bias * sum(x)
    float xo[ITERS];
#pragma unroll
    for (int it = 0; it < ITERS; it++) xo[it] = -OFF * xs[it];

    // one pass: the rows of bbase from register set Q
    auto pass = [&](auto bufc, uint32_t bbase) {
        constexpr int Q = decltype(bufc)::value;
        const uint32_t row0 = bbase + lane_row;
        float part[RPW];
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            part[r] = 0.0f;
#pragma unroll
            for (int it = 0; it < ITERS; it++) {
                const float sc = SB_F16 ? f16_to_f32(sh[Q][r][it]) : bf16_to_f32(sh[Q][r][it]);
                const float bi = SB_F16 ? f16_to_f32(bh[Q][r][it]) : bf16_to_f32(bh[Q][r][it]);
                float d = xo[it];
                d = word_dot(wv[Q][r][it].x, &xp[it][0], d);
                d = word_dot(wv[Q][r][it].y, &xp[it][4], d);
                d = word_dot(wv[Q][r][it].z, &xp[it][8], d);
                d = word_dot(wv[Q][r][it].w, &xp[it][12], d);
                part[r] = fmaf(sc, d, part[r]);
                part[r] = fmaf(bi, xs[it], part[r]);
            }
        }
        slice_sums_last<LPR, RPW>(part);
        if constexpr (KSPLIT > 1) {
            // K parts 1.. hand their slice totals to part 0 through LDS
            const int slot = (rg * SLICES + slice) * RPW;
            if (ks > 0 && sl == LPR - 1)
#pragma unroll
                for (int r = 0; r < RPW; r++)
                    red[((ks - 1) * RGROUPS * SLICES * RPW) + slot + r] = part[r];
            __syncthreads();
            if (ks == 0 && sl == LPR - 1)
#pragma unroll
                for (int k = 1; k < KSPLIT; k++)
#pragma unroll
                    for (int r = 0; r < RPW; r++)
                        part[r] += red[((k - 1) * RGROUPS * SLICES * RPW) + slot + r];
            __syncthreads();
        }
        if constexpr (PRO == PRO_RMSNORM || PRO == PRO_NORMED) {
            // the K parts' sums of squares are in LDS since the exchange above
            float tot = ss_part;
            if constexpr (KSPLIT > 1) {
                tot = 0.0f;
#pragma unroll
                for (int k = 0; k < KSPLIT; k++) tot += ssq[rg * KSPLIT + k];
            }
            const float inv = 1.0f / (float)sqrt((double)(tot / (float)K + fu.eps));
#pragma unroll
            for (int r = 0; r < RPW; r++) part[r] *= inv;
        }
        if (ks == 0 && sl == LPR - 1) {
            if constexpr (EPI == EPI_RESID) {
#pragma unroll
                for (int r = 0; r < RPW; r++)
                    if (row0 + r < N) static_cast<float*>(Y)[row0 + r] = rv[Q][r] + part[r];
            } else if constexpr (EPI == EPI_RESID_NORM) {
#pragma unroll
                for (int r = 0; r < RPW; r++)
                    if (row0 + r < N) {
                        const float h = rv[Q][r] + part[r];
                        static_cast<float*>(Y)[row0 + r] = h;
                        fu.nout[row0 + r] = f32_to_bf16_hw(h * bf16_to_f32(nv[Q][r]));
                        sq = fmaf(h, h, sq);
                    }
            } else if constexpr (EPI == EPI_SWIGLU) {
                float act[RO];
#pragma unroll
                // SiLU with the hardware exp (v_exp_f32, a few ulp, far inside the
                // product's tolerance): a double exp's dependent chain held the
                // storing lanes up longer than the rest of the epilogue
                for (int r = 0; r < RO; r++) act[r] = part[r] / (1.0f + __expf(-part[r])) * part[RO + r];
                store_rows<RO>(Y, y_dt, row0, N, act);
            } else {
                store_rows<RPW>(Y, y_dt, row0, N, part);
            }
        }
    };
    if constexpr (!PIPE) {
        for (uint32_t blk = blk0; blk < nblk; blk += bstride) {
            const uint32_t bbase = rmap.base(blk);
            if (blk != blk0) load_pass(B0{}, bbase + lane_row);
            pass(B0{}, bbase);
        }
    } else {
        // set 0 holds the first pass; each pass requests the one after it into
        // the other set before computing (the trip count is uniform over the block)
        for (uint32_t blk = blk0; blk < nblk; blk += 2 * bstride) {
            const uint32_t b1 = blk + bstride;
            if (b1 < nblk) load_pass(B1{}, rmap.base(b1) + lane_row);
            pass(B0{}, rmap.base(blk));
            if (b1 >= nblk) break;
            if (b1 + bstride < nblk) load_pass(B0{}, rmap.base(b1 + bstride) + lane_row);
            pass(B1{}, rmap.base(b1));
        }
    }
    if constexpr (EPI == EPI_RESID_NORM) {
        // this block's partial of the sum of y^2 (lanes that stored no row hold 0)
        __shared__ float bsum[4];
        const float w = wave_sum(sq);
        if (lane == 0) bsum[wv_id] = w;
        __syncthreads();
        if (threadIdx.x == 0) fu.stats[blockIdx.x] = (bsum[0] + bsum[1]) + (bsum[2] + bsum[3]);
        if (blockIdx.x == 0)
            for (int i = gridDim.x + threadIdx.x; i < kNormSlots; i += 256) fu.stats[i] = 0.0f;
    }
}

// The plain decode product: the grid strides over consecutive row blocks.
template <int LPR, int ITERS, int RPW, int KSPLIT, bool SB_F16, int PRO = PRO_NONE, int EPI = EPI_STORE,
          int BITS = 4, bool PIPE = false>
__global__ __launch_bounds__(256) void qmv_bf16x_kernel(
    const uint32_t* __restrict__ W, const uint16_t* __restrict__ S,
    const uint16_t* __restrict__ B, const void* __restrict__ Xv, void* Y,
    int y_dt, uint32_t N, int gs_log2, QmvFusion fu) {
    constexpr uint32_t RPB = qmv_rows_per_block<LPR, RPW, KSPLIT, EPI>();
    qmv_tile<LPR, ITERS, RPW, KSPLIT, SB_F16, PRO, EPI, BITS, PIPE>(W, S, B, Xv, Y, y_dt, N, gs_log2, fu, blockIdx.x,
                                                                    gridDim.x, (N + RPB - 1) / RPB, LinearRows{RPB});
}

}  // namespace qmvt
}  // namespace jh
