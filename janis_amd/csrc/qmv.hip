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
//  * Codes become bf16 without conversion instructions: a code q in the low 4
//    mantissa bits of bf16(128.0) = 0x4300 is exactly 128 + q. Two masks split a
//    word into its even and odd codes (one per byte) and v_perm_b32 assembles
//    the pairs (128 + q_p, 128 + q_{p+4}). v_dot2_f32_bf16 multiplies a pair
//    with the bf16 pair (x_p, x_{p+4}) and accumulates in fp32, so 8 codes cost
//    7 integer ops and 4 dot2. The constant 128 is removed through the x-sum
//    that the factorisation needs anyway: each dot product starts from
//    -128*sum(x), so it ends at sum(x*(128+q)) - 128*sum(x) = sum(x*q), and a
//    group costs two fma beyond it: scale*dot + bias*sum(x).
//  * Partial sums are reduced across the slice with cross-lane adds; the
//    slice's first lane writes y (fp32 or bf16).
#include "qmv_tile.hpp"

namespace jh {
using namespace qmvt;
namespace {

// A few rows of x (2..MR) through the decode tile: each weight word is loaded
// and split into (128 + q) bf16 pairs once and applied to every row's x, so
// the weights stream from HBM once for all rows. The lanes, words, dot order
// and reductions are those of qmv_bf16x_kernel with the same tile, so row m of
// y has the bits a one-row call on x[m] gives. x rows of bf16 (XF32: fp32,
// rounded to bf16 in registers as the one-row tile does) and y rows of N (bf16
// or fp32); rows past `rows` read as zero and are not stored.
template <int LPR, int ITERS, int RPW, int KSPLIT, bool SB_F16, int MR, bool XF32>
__global__ __launch_bounds__(256) void qmv_rows_kernel(
    const uint32_t* __restrict__ W, const uint16_t* __restrict__ S, const uint16_t* __restrict__ B,
    const void* __restrict__ X, void* Y, int y_dt, uint32_t N, int gs_log2, int rows) {
    constexpr int SLICES = 64 / LPR;
    constexpr int RGROUPS = 4 / KSPLIT;
    constexpr uint32_t PK = 4 * LPR * ITERS;
    constexpr uint32_t P = PK * KSPLIT;
    constexpr uint32_t K = 8 * P;
    constexpr int ROWS_PER_WAVE = SLICES * RPW;
    constexpr int ROWS_PER_BLOCK = RGROUPS * ROWS_PER_WAVE;
    const int lane = threadIdx.x & 63;
    const int wv_id = threadIdx.x >> 6;
    const int ks = wv_id % KSPLIT, rg = wv_id / KSPLIT;
    const int sl = lane % LPR, slice = lane / LPR;
    const uint32_t G = K >> gs_log2;
    const auto rw = make_rsrc(W, N * P * 4);
    const auto rs = make_rsrc(S, N * G * 2);
    const auto rb = make_rsrc(B, N * G * 2);
    constexpr uint32_t XB = XF32 ? 4 : 2;  // bytes per x element
    const auto rx = make_rsrc(X, (uint32_t)rows * K * XB);
    __shared__ float red[(KSPLIT > 1) ? (KSPLIT - 1) * RGROUPS * SLICES * RPW * MR : 1];

    uint32_t gi[ITERS], wo[ITERS];
#pragma unroll
    for (int it = 0; it < ITERS; it++) {
        wo[it] = ks * PK + it * 4 * LPR + 4 * sl;
        gi[it] = (8 * wo[it]) >> gs_log2;
    }
    // every row's part of x as (x_p, x_{p+4}) pairs, and its group sums
    uint32_t xp[MR][ITERS][16];
    float xs[MR][ITERS];
    if constexpr (XF32) {
        // fp32 rows: each wave reads its K part of a row with consecutive lanes
        // on consecutive 16 bytes, rounds it to bf16 (nearest even) into LDS and
        // takes its runs from there (as the one-row tile does), row after row
        constexpr uint32_t XE = 8 * PK;  // elements of a wave's K part
        constexpr int XC = (int)((XE / 4 + 63) / 64);
        __shared__ uint2 xstage[4 * (XE / 4)];
        uint2* xw = xstage + wv_id * (XE / 4);
        auto cvt2 = [](uint32_t u, uint32_t v) {
            return (uint32_t)f32_to_bf16_hw(__uint_as_float(u)) | ((uint32_t)f32_to_bf16_hw(__uint_as_float(v)) << 16);
        };
#pragma unroll
        for (int m = 0; m < MR; m++) {
            const uint32_t base = (m * K + ks * XE) * 4;
            u32x4_t c4[XC];
#pragma unroll
            for (int c = 0; c < XC; c++)
                c4[c] = __builtin_amdgcn_raw_buffer_load_b128(rx, base + (uint32_t)(c * 64 + lane) * 16, 0, 0);
            if (m > 0) __syncthreads();  // the previous row's runs are read
#pragma unroll
            for (int c = 0; c < XC; c++)
                if ((uint32_t)(c * 64 + lane) < XE / 4)
                    xw[c * 64 + lane] = make_uint2(cvt2(c4[c].x, c4[c].y), cvt2(c4[c].z, c4[c].w));
            __syncthreads();
#pragma unroll
            for (int it = 0; it < ITERS; it++) {
                const uint4* src = reinterpret_cast<const uint4*>(xw + (8 * (wo[it] - ks * PK)) / 4);
                float sum = 0.0f;
#pragma unroll
                for (int j = 0; j < 4; j++) sum += pair_up(src[j], &xp[m][it][4 * j]);
                xs[m][it] = sum;
            }
        }
    } else {
#pragma unroll
        for (int m = 0; m < MR; m++)
#pragma unroll
            for (int it = 0; it < ITERS; it++) {
                const uint32_t off = (m * K + 8 * wo[it]) * 2;
                float sum = 0.0f;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rx, off + 16 * j, 0, 0);
                    sum += pair_up(make_uint4(v.x, v.y, v.z, v.w), &xp[m][it][4 * j]);
                }
                xs[m][it] = sum;
            }
    }

    const uint32_t lane_row = rg * ROWS_PER_WAVE + (uint32_t)slice * RPW;
    for (uint32_t bbase = blockIdx.x * ROWS_PER_BLOCK; bbase < N; bbase += gridDim.x * ROWS_PER_BLOCK) {
        const uint32_t row0 = bbase + lane_row;
        uint4 wv[RPW][ITERS];
        uint16_t sh[RPW][ITERS], bh[RPW][ITERS];
#pragma unroll
        for (int r = 0; r < RPW; r++)
#pragma unroll
            for (int it = 0; it < ITERS; it++) wv[r][it] = buf_load16_nt(rw, ((row0 + r) * P + wo[it]) * 4);
#pragma unroll
        for (int r = 0; r < RPW; r++)
#pragma unroll
            for (int it = 0; it < ITERS; it++) {
                const uint32_t off = ((row0 + r) * G + gi[it]) * 2;
                sh[r][it] = buf_load2(rs, off);
                bh[r][it] = buf_load2(rb, off);
            }
        float part[MR * RPW];
#pragma unroll
        for (int i = 0; i < MR * RPW; i++) part[i] = 0.0f;
#pragma unroll
        for (int r = 0; r < RPW; r++)
#pragma unroll
            for (int it = 0; it < ITERS; it++) {
                const float sc = SB_F16 ? f16_to_f32(sh[r][it]) : bf16_to_f32(sh[r][it]);
                const float bi = SB_F16 ? f16_to_f32(bh[r][it]) : bf16_to_f32(bh[r][it]);
                float d[MR];  // from -128 * sum(x), as the one-row tile starts them
#pragma unroll
                for (int m = 0; m < MR; m++) d[m] = -kCodeOffset * xs[m][it];
                const uint32_t words[4] = {wv[r][it].x, wv[r][it].y, wv[r][it].z, wv[r][it].w};
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const uint32_t lo = words[q] & 0x0F0F0F0Fu;
                    const uint32_t hi = (words[q] >> 4) & 0x0F0F0F0Fu;
                    const uint32_t c0 = __builtin_amdgcn_perm(kBf16Bytes, lo, kSelB0B2);
                    const uint32_t c1 = __builtin_amdgcn_perm(kBf16Bytes, hi, kSelB0B2);
                    const uint32_t c2 = __builtin_amdgcn_perm(kBf16Bytes, lo, kSelB1B3);
                    const uint32_t c3 = __builtin_amdgcn_perm(kBf16Bytes, hi, kSelB1B3);
#pragma unroll
                    for (int m = 0; m < MR; m++) {
                        d[m] = dot2_bf16(c0, xp[m][it][4 * q + 0], d[m]);
                        d[m] = dot2_bf16(c1, xp[m][it][4 * q + 1], d[m]);
                        d[m] = dot2_bf16(c2, xp[m][it][4 * q + 2], d[m]);
                        d[m] = dot2_bf16(c3, xp[m][it][4 * q + 3], d[m]);
                    }
                }
#pragma unroll
                for (int m = 0; m < MR; m++) {
                    part[m * RPW + r] = fmaf(sc, d[m], part[m * RPW + r]);
                    part[m * RPW + r] = fmaf(bi, xs[m][it], part[m * RPW + r]);
                }
            }
        slice_sums_last<LPR, MR * RPW>(part);
        if constexpr (KSPLIT > 1) {
            const int slot = (rg * SLICES + slice) * RPW * MR;
            if (ks > 0 && sl == LPR - 1)
#pragma unroll
                for (int i = 0; i < MR * RPW; i++) red[((ks - 1) * RGROUPS * SLICES * RPW * MR) + slot + i] = part[i];
            __syncthreads();
            if (ks == 0 && sl == LPR - 1)
#pragma unroll
                for (int k = 1; k < KSPLIT; k++)
#pragma unroll
                    for (int i = 0; i < MR * RPW; i++) part[i] += red[((k - 1) * RGROUPS * SLICES * RPW * MR) + slot + i];
            __syncthreads();
        }
        if (ks == 0 && sl == LPR - 1) {
#pragma unroll
            for (int m = 0; m < MR; m++)
                if (m < rows)
#pragma unroll
                    for (int r = 0; r < RPW; r++)
                        if (row0 + r < N) {
                            const size_t o = (size_t)m * N + row0 + r;
                            if (y_dt == JH_BF16)
                                static_cast<uint16_t*>(Y)[o] = f32_to_bf16_hw(part[m * RPW + r]);
                            else
                                static_cast<float*>(Y)[o] = part[m * RPW + r];
                        }
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
    int64_t K, int gs, int bits, int64_t M, const int* __restrict__ ws, int64_t n_experts,
    int64_t k_slots, int64_t a_vectors) {
    const int lane = threadIdx.x & 63;
    const int vpw = 32 / bits;
    const uint32_t mask = (1u << bits) - 1u;
    const int64_t P = K / vpw, G = K / gs;
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
                for (int l = 0; l < vpw; l++) {
                    const int64_t j = vpw * p + l;
                    const int64_t g = j / gs;
                    const float s = load_sb(S, sb0 + row * G + g, sb_dt);
                    const float b = load_sb(B, sb0 + row * G + g, sb_dt);
                    const float w = fmaf((float)((word >> (bits * l)) & mask), s, b);
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

// BPC > 0: the pipelined kernel on a grid of at most BPC blocks per CU.
template <int LPR, int ITERS, int RPW, int KSPLIT, bool SB_F16, int PRO = PRO_NONE, int EPI = EPI_STORE,
          int BITS = 4, int BPC = 0>
Status run_fast_sb(const QuantMatrix& m, const void* x, void* y, int y_dtype, int gs_log2,
                   int num_cus, hipStream_t st, const QmvFusion& fu = QmvFusion{}) {
    constexpr int64_t rows_per_block = (4 / KSPLIT) * (64 / LPR) * (EPI == EPI_SWIGLU ? RPW / 2 : RPW);
    // the tile's row length must be the matrix's: the kernel sizes its buffer
    // resources and group offsets from it
    constexpr int64_t k_tile = 4LL * LPR * ITERS * KSPLIT * (32 / BITS);
    if (k_tile != m.in || m.bits != BITS) return Status::fail(JH_ERR_UNSUPPORTED, "qmv: tile does not fit the matrix");
    const int64_t n_out = EPI == EPI_SWIGLU ? m.rows / 2 : m.rows;
    auto kern = qmv_bf16x_kernel<LPR, ITERS, RPW, KSPLIT, SB_F16, PRO, EPI, BITS, (BPC > 0)>;
    // persistent-style grid: at most what is resident at once, so multi-pass
    // shapes reuse the x registers instead of queueing more blocks
    static int resident = 0;
    if (resident == 0) {
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, 256, 0) != hipSuccess || per_cu < 1)
            per_cu = 2;
        resident = per_cu;
    }
    int64_t blocks = (n_out + rows_per_block - 1) / rows_per_block;
    const int64_t cap = (int64_t)num_cus * (BPC > 0 ? BPC : resident);
    if (blocks > cap) blocks = cap;
    if (EPI == EPI_RESID_NORM && blocks > kNormSlots) blocks = kNormSlots;  // one partial per block
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), 0, st, m.w,
                       static_cast<const uint16_t*>(m.scales), static_cast<const uint16_t*>(m.biases), x, y,
                       y_dtype, (uint32_t)n_out, gs_log2, fu);
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
                       m.group_size, m.bits, rows, nullptr, (int64_t)1, (int64_t)1, (int64_t)1);
    return Status::ok();
}

namespace {

// One tile of the table. Fused prologues/epilogues are built for bf16 scales
// only (the checkpoints' format); an f16-scale fused call returns false and is
// composed from separate launches by the caller.
template <int LPR, int ITERS, int RPW, int KSPLIT, int PRO, int EPI, int BITS, int BPC>
bool tile_bits(const QuantMatrix& m, const void* x, void* y, int y_dtype, int gl, int num_cus, hipStream_t st,
               const QmvFusion& fu) {
    if (m.sb_dtype == JH_F16) {
        if constexpr ((PRO == PRO_NONE || PRO == PRO_XF32) && EPI == EPI_STORE)
            return run_fast_sb<LPR, ITERS, RPW, KSPLIT, true, PRO, EPI, BITS, BPC>(m, x, y, y_dtype, gl, num_cus, st,
                                                                                 fu)
                       .code == JH_OK;
        else
            return false;
    }
    return run_fast_sb<LPR, ITERS, RPW, KSPLIT, false, PRO, EPI, BITS, BPC>(m, x, y, y_dtype, gl, num_cus, st, fu)
               .code == JH_OK;
}

// 8-bit weights have tiles for a plain or prepared-norm bf16 input.
template <int LPR, int ITERS, int RPW, int KSPLIT, int PRO, int EPI, int BPC = 0>
bool tile(const QuantMatrix& m, const void* x, void* y, int y_dtype, int gl, int num_cus, hipStream_t st,
          const QmvFusion& fu) {
    if (m.bits == 8) {
        if constexpr (PRO == PRO_RMSNORM) return false;
        else return tile_bits<LPR, ITERS, RPW, KSPLIT, PRO, EPI, 8, BPC>(m, x, y, y_dtype, gl, num_cus, st, fu);
    }
    return tile_bits<LPR, ITERS, RPW, KSPLIT, PRO, EPI, 4, BPC>(m, x, y, y_dtype, gl, num_cus, st, fu);
}

// The register tiles take 4- and 8-bit weights, groups of 32/64/128 dividing K,
// 16-bit scales, matrices under 2 GiB and the row lengths P (words) of the
// table below: K = 8P for 4-bit, 4P for 8-bit.
int64_t row_words(const QuantMatrix& m) { return m.in * m.bits / 32; }

bool qmv_fast_shape(const QuantMatrix& m) {
    const int gl = log2_exact(m.group_size);
    if (!((m.bits == 4 || m.bits == 8) && gl >= 5 && gl <= 7 && (m.in % m.group_size) == 0 &&
          (m.in % (32 / m.bits)) == 0 && (m.sb_dtype == JH_BF16 || m.sb_dtype == JH_F16) &&
          (m.rows + 64) * row_words(m) * 4 < ((int64_t)1 << 31)))
        return false;
    switch (row_words(m)) {
        case 512: case 1024: case 1536: case 2048: case 3072: case 256: case 768:
        case 128: case 384: case 64: case 192: case 32: case 96:
            return true;
        default:
            return false;
    }
}

// Tile per row length, from sweeps of the Qwen3-8B shapes on MI355X (graph
// replays over weight copies that do not fit the last-level cache): splitting
// K over 2-4 waves per row beats one wave per row at every shape (more waves in
// flight, shorter per-wave dependency chains). For 512-word rows, matrices of
// up to 4096 output rows take 2 rows per slice (twice the blocks: o_proj 4.16
// against 4.37 us) and larger ones 4 (gate+up 11.6 against 12.4 us; the
// 151936-row lm_head 57.0 us, against 63.5 for a 64-lane 2-way tile). Rows of
// 1536 words (down_proj, K = 12288) take one row per slice on a grid of two
// blocks per CU, each block walking four passes with the next pass's loads in
// flight while it computes (7.65 against 8.29 us at 4096 rows): with a whole
// row's three 16-byte loads per lane issued at once, the single-pass tile
// waits for all of its loads before any dot product starts.
template <int PRO, int EPI>
bool launch_tiles(const QuantMatrix& m, const void* x, void* y, int y_dtype, int num_cus, hipStream_t st,
                  const QmvFusion& fu) {
    if (!qmv_fast_shape(m)) return false;
    const int gl = log2_exact(m.group_size);
    const int64_t n_out = EPI == EPI_SWIGLU ? m.rows / 2 : m.rows;
#define JH_TILE(L, I, R, KS) return tile<L, I, R, KS, PRO, EPI>(m, x, y, y_dtype, gl, num_cus, st, fu)
    switch (row_words(m)) {
        case 512 * 1:
            if (n_out <= 4096 && EPI != EPI_SWIGLU) JH_TILE(32, 1, 2, 4);
            JH_TILE(32, 1, 4, 4);
        case 512 * 2: JH_TILE(32, 2, 2, 4);
        case 512 * 3:
            if constexpr (EPI != EPI_SWIGLU)
                if (n_out >= 2048) return tile<32, 3, 1, 4, PRO, EPI, 2>(m, x, y, y_dtype, gl, num_cus, st, fu);
            JH_TILE(32, 3, 2, 4);
        case 512 * 4: JH_TILE(32, 4, 2, 4);
        case 512 * 6: JH_TILE(64, 3, 2, 4);  // 8-bit K = 12288
        case 256 * 1: JH_TILE(32, 1, 4, 2);
        case 256 * 3: JH_TILE(32, 3, 2, 2);
        case 128 * 1: JH_TILE(16, 1, 4, 2);
        case 128 * 3: JH_TILE(16, 3, 2, 2);
        case 64 * 1: JH_TILE(16, 1, 4, 1);
        case 64 * 3: JH_TILE(16, 3, 2, 1);
        case 32 * 1: JH_TILE(8, 1, 4, 1);
        case 32 * 3: JH_TILE(8, 3, 2, 1);
        default: return false;
    }
#undef JH_TILE
}

}  // namespace

Status launch_qmv(const QuantMatrix& m, const void* x, int x_dtype, void* y, int y_dtype,
                  int num_cus, hipStream_t st) {
    if (x_dtype == JH_BF16 && launch_tiles<PRO_NONE, EPI_STORE>(m, x, y, y_dtype, num_cus, st, QmvFusion{}))
        return Status::ok();
    // fp32 x (the CPU backend's activation type): the same tiles, x rounded to
    // bf16 in registers
    if (x_dtype == JH_F32 && launch_tiles<PRO_XF32, EPI_STORE>(m, x, y, y_dtype, num_cus, st, QmvFusion{}))
        return Status::ok();
    return launch_generic(m, x, x_dtype, 1, y, y_dtype, num_cus, st);
}


namespace {

// Rows of x per launch of the multi-row tile: x of MR rows lives in registers
// (16 VGPRs per row and 32 elements of a lane's K part), so long K parts take
// fewer rows per launch.
template <int ITERS>
constexpr int rows_mr() { return ITERS == 1 ? 8 : (ITERS == 2 ? 4 : 2); }

template <int LPR, int ITERS, int RPW, int KSPLIT, bool SB_F16, int MR, bool XF32>
Status run_rows_mr(const QuantMatrix& m, const void* x, int64_t rows, void* y, int y_dtype, int gl,
                   int num_cus, hipStream_t st) {
    constexpr int64_t rows_per_block = (4 / KSPLIT) * (64 / LPR) * RPW;
    constexpr size_t xsz = XF32 ? 4 : 2;
    auto kern = qmv_rows_kernel<LPR, ITERS, RPW, KSPLIT, SB_F16, MR, XF32>;
    static int per_cu = 0;  // resident blocks per CU, asked once per instantiation
    if (per_cu == 0 && (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, 256, 0) != hipSuccess || per_cu < 1))
        per_cu = 1;
    int64_t blocks = (m.rows + rows_per_block - 1) / rows_per_block;
    blocks = std::max<int64_t>(1, std::min<int64_t>(blocks, (int64_t)num_cus * per_cu));
    const size_t ysz = y_dtype == JH_BF16 ? 2 : 4;
    for (int64_t r0 = 0; r0 < rows; r0 += MR) {
        const int n = (int)std::min<int64_t>(MR, rows - r0);
        hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), 0, st, m.w,
                           static_cast<const uint16_t*>(m.scales), static_cast<const uint16_t*>(m.biases),
                           static_cast<const char*>(x) + (size_t)r0 * m.in * xsz,
                           static_cast<char*>(y) + (size_t)r0 * m.rows * ysz, y_dtype,
                           (uint32_t)m.rows, gl, n);
    }
    return Status::ok();
}

// The kernel computes all MR rows whatever the count, so the smallest of 2, 4
// and 8 rows per launch that covers the call (up to the tile's limit) is used.
template <int LPR, int ITERS, int RPW, int KSPLIT, bool SB_F16, bool XF32>
Status run_rows(const QuantMatrix& m, const void* x, int64_t rows, void* y, int y_dtype, int gl, int num_cus,
                hipStream_t st) {
    constexpr int MRMAX = rows_mr<ITERS>();
    if constexpr (MRMAX >= 8)
        if (rows > 4)
            return run_rows_mr<LPR, ITERS, RPW, KSPLIT, SB_F16, 8, XF32>(m, x, rows, y, y_dtype, gl, num_cus, st);
    if constexpr (MRMAX >= 4)
        if (rows > 2)
            return run_rows_mr<LPR, ITERS, RPW, KSPLIT, SB_F16, 4, XF32>(m, x, rows, y, y_dtype, gl, num_cus, st);
    return run_rows_mr<LPR, ITERS, RPW, KSPLIT, SB_F16, 2, XF32>(m, x, rows, y, y_dtype, gl, num_cus, st);
}

template <int LPR, int ITERS, int RPW, int KSPLIT>
Status run_rows_dt(const QuantMatrix& m, const void* x, int x_dtype, int64_t rows, void* y, int y_dtype, int gl,
                   int num_cus, hipStream_t st) {
    const bool f16 = m.sb_dtype == JH_F16;
    if (x_dtype == JH_F32)
        return f16 ? run_rows<LPR, ITERS, RPW, KSPLIT, true, true>(m, x, rows, y, y_dtype, gl, num_cus, st)
                   : run_rows<LPR, ITERS, RPW, KSPLIT, false, true>(m, x, rows, y, y_dtype, gl, num_cus, st);
    return f16 ? run_rows<LPR, ITERS, RPW, KSPLIT, true, false>(m, x, rows, y, y_dtype, gl, num_cus, st)
               : run_rows<LPR, ITERS, RPW, KSPLIT, false, false>(m, x, rows, y, y_dtype, gl, num_cus, st);
}

// 16-byte weight loads per lane and row of the multi-row tile for a 4-bit row
// length, or 0 when no multi-row tile takes it.
int tile_iters(int64_t row_words) {
    switch (row_words) {
        case 512 * 1: case 256 * 1: case 128 * 1: case 64 * 1: case 32 * 1: return 1;
        case 512 * 2: return 2;
        case 512 * 3: case 256 * 3: case 128 * 3: case 64 * 3: case 32 * 3: case 512 * 6: return 3;
        case 512 * 4: return 4;
        default: return 0;
    }
}

}  // namespace

// Which few-row calls the multi-row tile takes, and which go to the prefill
// GEMM, from graph-replay timings on MI355X over weight copies that do not fit
// the memory-side cache. The tile reads the weights once and does all the rows'
// dot products in VALU, so it wins while the matrix is small and loses on large
// ones once the rows multiply its arithmetic:
//  * 2 rows: always the tile;
//  * 3-4 rows: the tile for 16-byte-load tiles (K = 256..8192 in this table);
//    for tiles whose lanes hold 96 or 128 elements of a row only from K = 1536
//    and below 16M weights (4096 x 1536 at 4 rows 9.4 us against 10.6 for the
//    GEMM, 1024 x 3072 9.3 against 9.4; 2048 x 768 9.1 against 6.7, 4096 x
//    6144 14.7 against 11.9, 4096 x 12288 22.3 against 15.9);
//  * 5-8 rows: the tile from K = 1024 below 16M weights (1024 x 4096 at 5 rows
//    7.6 against 9.3 us, 8192 x 1024 7.3 against 8.2), the GEMM from 16M
//    weights (4096 x 4096 at 8 rows 11.7 against 10.6, 12288 x 4096 23.3
//    against 17.8, 24576 x 4096 40.7 against 24.8) and at K = 512 (4096 x 512
//    6.9 against 5.6).
// Only row lengths with a case in launch_qmv_rows are accepted (tile_iters > 0).
bool qmv_rows_ok(const QuantMatrix& m, int64_t rows, int x_dtype) {
    if ((x_dtype != JH_BF16 && x_dtype != JH_F32) || m.bits != 4 || rows < 2 || !qmv_fast_shape(m) ||
        rows * m.in * 4 >= ((int64_t)1 << 31))
        return false;
    const int it = tile_iters(row_words(m));
    if (it == 0 || rows > kQmvRowsMax) return false;
    if (rows == 2) return true;
    constexpr int64_t kSmallWeights = (int64_t)1 << 24;
    const bool small = m.rows * m.in < kSmallWeights;
    if (it >= 3) return rows <= 4 && small && m.in >= 1536;
    return rows <= 4 || (small && m.in >= 1024);
}

Status launch_qmv_rows(const QuantMatrix& m, const void* x, int x_dtype, int64_t rows, void* y, int y_dtype,
                       int num_cus, hipStream_t st) {
    if (!qmv_rows_ok(m, rows, x_dtype)) return Status::fail(JH_ERR_UNSUPPORTED, "qmv_rows: shape outside the tiles");
    const int gl = log2_exact(m.group_size);
#define JH_ROWS(L, I, R, KS) return run_rows_dt<L, I, R, KS>(m, x, x_dtype, rows, y, y_dtype, gl, num_cus, st)
    // Each case keeps the one-row tile's lanes per row (L), loads per lane (I)
    // and K split (KS) for that row length, so a row's reduction order -- and
    // its bits -- are those of a one-row call; only the rows per slice (R) may
    // differ.
    switch (row_words(m)) {
        case 512 * 1: JH_ROWS(32, 1, 4, 4);
        case 512 * 2: JH_ROWS(32, 2, 2, 4);
        case 512 * 3: JH_ROWS(32, 3, 2, 4);
        case 512 * 4: JH_ROWS(32, 4, 2, 4);
        case 512 * 6: JH_ROWS(64, 3, 2, 4);
        case 256 * 1: JH_ROWS(32, 1, 4, 2);
        case 256 * 3: JH_ROWS(32, 3, 2, 2);
        case 128 * 1: JH_ROWS(16, 1, 4, 2);
        case 128 * 3: JH_ROWS(16, 3, 2, 2);
        case 64 * 1: JH_ROWS(16, 1, 4, 1);
        case 64 * 3: JH_ROWS(16, 3, 2, 1);
        case 32 * 1: JH_ROWS(8, 1, 4, 1);
        case 32 * 3: JH_ROWS(8, 3, 2, 1);
        default: return Status::fail(JH_ERR_UNSUPPORTED, "qmv_rows: no tile for the row length");
    }
#undef JH_ROWS
}

// True when one register-tile launch takes the fused call (no workspace).
bool qmv_fused_single(const QuantMatrix& m, int pro, int x_dtype, int nw_dtype, int epi, int y_dtype) {
    if (pro == PRO_RMSNORM ? (x_dtype != JH_F32 || nw_dtype != JH_BF16)
                           : ((pro != PRO_NONE && pro != PRO_NORMED) || x_dtype != JH_BF16))
        return false;
    if ((epi == EPI_RESID || epi == EPI_RESID_NORM) && y_dtype != JH_F32) return false;
    if (epi == EPI_RESID_NORM && nw_dtype != JH_BF16) return false;
    if (!qmv_fast_shape(m)) return false;
    if (m.bits == 8 && pro == PRO_RMSNORM) return false;
    if (m.sb_dtype != JH_BF16 && (pro != PRO_NONE || epi != EPI_STORE)) return false;
    if (pro == PRO_NONE) return epi == EPI_STORE || epi == EPI_RESID || epi == EPI_RESID_NORM;
    return epi == EPI_STORE || epi == EPI_SWIGLU;
}

size_t qmv_fused_workspace_bytes(const QuantMatrix& m, int pro, int x_dtype, int nw_dtype, int epi, int y_dtype) {
    if (qmv_fused_single(m, pro, x_dtype, nw_dtype, epi, y_dtype)) return 0;
    return ((size_t)m.in * 2 + 255) / 256 * 256 + (size_t)m.rows * 4;
}

Status launch_qmv_fused(const QuantMatrix& m, int pro, const void* x, int x_dtype, const void* nw, int nw_dtype,
                        float eps, int epi, const float* resid, void* y, int y_dtype, const NormSplit& ns,
                        int num_cus, hipStream_t st, void* workspace) {
    // one launch when a register tile takes the shape
    if (qmv_fused_single(m, pro, x_dtype, nw_dtype, epi, y_dtype)) {
        QmvFusion fu;
        fu.nw = static_cast<const uint16_t*>(nw);
        fu.eps = eps;
        fu.resid = resid;
        fu.stats = ns.stats;
        fu.nout = ns.out;
        bool done = false;
        if (pro == PRO_NONE && epi == EPI_STORE)
            done = launch_tiles<PRO_NONE, EPI_STORE>(m, x, y, y_dtype, num_cus, st, fu);
        else if (pro == PRO_NONE && epi == EPI_RESID)
            done = launch_tiles<PRO_NONE, EPI_RESID>(m, x, y, y_dtype, num_cus, st, fu);
        else if (pro == PRO_NONE)
            done = launch_tiles<PRO_NONE, EPI_RESID_NORM>(m, x, y, y_dtype, num_cus, st, fu);
        else if (pro == PRO_RMSNORM && epi == EPI_STORE)
            done = launch_tiles<PRO_RMSNORM, EPI_STORE>(m, x, y, y_dtype, num_cus, st, fu);
        else if (pro == PRO_RMSNORM)
            done = launch_tiles<PRO_RMSNORM, EPI_SWIGLU>(m, x, y, y_dtype, num_cus, st, fu);
        else if (epi == EPI_STORE)
            done = launch_tiles<PRO_NORMED, EPI_STORE>(m, x, y, y_dtype, num_cus, st, fu);
        else
            done = launch_tiles<PRO_NORMED, EPI_SWIGLU>(m, x, y, y_dtype, num_cus, st, fu);
        if (done) return Status::ok();
        return Status::fail(JH_ERR_UNSUPPORTED, "qmv_fused: no tile for a shape the planner accepted");
    }
    // otherwise the same arithmetic as separate launches through the workspace
    if (!workspace) return Status::fail(JH_ERR_INVALID, "qmv_fused: this combination needs a workspace");
    uint16_t* xin = static_cast<uint16_t*>(workspace);
    float* tmp = reinterpret_cast<float*>(static_cast<char*>(workspace) + ((size_t)m.in * 2 + 255) / 256 * 256);
    const void* xp = x;
    int xdt = x_dtype;
    if (pro == PRO_RMSNORM) {
        Status s = launch_rms_norm(x, x_dtype, nw, nw_dtype, eps, xin, JH_BF16, 1, m.in, st);
        if (s.code != JH_OK) return s;
        xp = xin, xdt = JH_BF16;
    } else if (pro == PRO_NORMED) {
        if (x_dtype != JH_BF16) return Status::fail(JH_ERR_INVALID, "qmv_fused: a prepared norm input is bf16");
        Status s = launch_norm_apply(static_cast<const uint16_t*>(x), m.in, ns.stats, eps, xin, st);
        if (s.code != JH_OK) return s;
        xp = xin, xdt = JH_BF16;
    } else if (pro == kProSiluMul) {
        const size_t esz = x_dtype == JH_F32 ? 4 : 2;
        Status s = launch_elementwise(JH_OP_SILU_MUL, x, x_dtype, static_cast<const char*>(x) + m.in * esz, x_dtype,
                                      xin, JH_BF16, m.in, st);
        if (s.code != JH_OK) return s;
        xp = xin, xdt = JH_BF16;
    }
    if (epi == EPI_STORE) return launch_qmv(m, xp, xdt, y, y_dtype, num_cus, st);
    Status s = launch_qmv(m, xp, xdt, tmp, JH_F32, num_cus, st);
    if (s.code != JH_OK) return s;
    if (epi == EPI_RESID) return launch_elementwise(JH_OP_ADD, resid, JH_F32, tmp, JH_F32, y, y_dtype, m.rows, st);
    if (epi == EPI_RESID_NORM) {
        s = launch_elementwise(JH_OP_ADD, resid, JH_F32, tmp, JH_F32, y, JH_F32, m.rows, st);
        if (s.code != JH_OK) return s;
        return launch_norm_prepare(y, JH_F32, m.rows, nw, nw_dtype, ns.out, ns.stats, st);
    }
    const int64_t n = m.rows / 2;
    return launch_elementwise(JH_OP_SILU_MUL, tmp, JH_F32, tmp + n, JH_F32, y, y_dtype, n, st);
}

}  // namespace jh
