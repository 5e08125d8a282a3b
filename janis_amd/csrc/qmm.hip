// Prefill GEMM for MLX affine 4-bit weights on gfx950:
//   Y[M, N] = X[M, K] . W^T.
// Three tiles share the MFMA layout below. K divisible by 256 takes a 128-row
// tile whose waves dequantize their own weight words into B fragments in
// registers: qmm_dma_kernel (X tiles, weight words and scales staged through
// LDS rings by loads with an LDS destination, several steps ahead; fp32 X is
// rounded to bf16 into the workspace first) and, where a lane's scales of a
// super-step do not fill whole dwords, qmm_wreg_kernel (weights prefetched in
// registers, X rounded on its way to LDS). Other K take qmm_mfma_kernel,
// described next, which dequantizes W tile by tile into LDS as bf16.
//
// Reference semantics: QuantMatmul with rows > 1 (cpu/cpu_misc.go:378-399),
// which dequantizes a weight row once (wbuf = q*scale + bias) and dots it with
// every x row in fp32. Here a block of 8 waves owns a 256x128 tile of Y and
// walks K in steps of 64:
//   * global -> registers: an X tile [256 x 64] (bf16; converted if X is fp32)
//     and a W tile [128 x 64] of packed words plus the group's scale and bias;
//   * registers -> LDS: W dequantized as fma(q, scale, bias) (exactly
//     fl32(q*scale+bias) for bf16/f16 scales) rounded to bf16; each dequantized
//     element feeds 256 rows of X, and the dequant of step k+1 is interleaved
//     with the MFMAs of step k;
//   * LDS -> MFMA: eight waves, each a 64x64 block of Y as 2x2
//     v_mfma_f32_32x32x16_bf16 tiles, fp32 accumulation.
// LDS is double-buffered (2 x 48 KiB; gfx950 has 160 KiB per CU) and the global
// loads run two steps ahead in registers; one barrier per step. Rows are stored unpadded with the 16-byte chunks
// XOR-swizzled by (row/2) % 8, so the 16-byte fragment reads of 16 consecutive
// rows hit 16 distinct bank groups.
// Operand layout of v_mfma_f32_32x32x16_bf16: lane l supplies
//   A[i = l % 32][k = 8*(l/32) .. +8]  and  B[k = 8*(l/32) .. +8][j = l % 32],
// and accumulator register r of lane l holds D[8*(r/4) + 4*(l/32) + r%4][l % 32].
// When the tile grid is too small to fill the GPU, K is split over blockIdx.z:
// each K range stores its fp32 partial tile and one pass adds them in order --
// inside the product's launch when its blocks are all resident at once
// (qmm_dma_kernel, INL), else a summing launch.
#include "jh_common.hpp"

namespace jh {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int BK = 64;
constexpr int ROW_BYTES = BK * 2;  // 128 B: 8 chunks of 16 B

// Byte offset of 16-byte chunk c of row r inside a [rows x 64] bf16 tile.
__device__ __forceinline__ uint32_t swz(int r, int c) {
    return r * ROW_BYTES + ((c ^ ((r >> 1) & 7)) << 4);
}

// Scale/bias element types: 0 bf16, 1 f16, 2 f32. The raw bits are loaded here
// and widened only when the stage is written to LDS, so no instruction waits on
// the prefetch loads before the MFMAs of the current step have been issued.
template <int SBT>
__device__ __forceinline__ uint32_t load_sb_bits(__amdgpu_buffer_rsrc_t r, uint32_t i) {
    if constexpr (SBT == 2)
        return __builtin_amdgcn_raw_buffer_load_b32(r, i * 4, 0, 0);
    else
        return buf_load2(r, i * 2);
}

template <int SBT>
__device__ __forceinline__ float widen_sb(uint32_t bits) {
    if constexpr (SBT == 2)
        return __uint_as_float(bits);
    else if constexpr (SBT == 1)
        return f16_to_f32((uint16_t)bits);
    else
        return bf16_to_f32((uint16_t)bits);
}

typedef float f32x2_t __attribute__((ext_vector_type(2)));

// One packed word -> 8 bf16 weights fl32(q*s + b) rounded to nearest even, in
// word order (q0 = lowest nibble): 3 masks, 8 v_cvt_f32_ubyteN, 8 FMAs and 4
// v_cvt_pk_bf16_f32.
__device__ __forceinline__ bf16x8_t dequant_word(uint32_t word, float sc, float bi) {
    uint32_t lo = word & 0x0F0F0F0Fu, hi = (word >> 4) & 0x0F0F0F0Fu;
    // An empty asm hides where lo and hi came from, so the byte extractions
    // below stay single v_cvt_f32_ubyteN instead of being re-derived as
    // per-nibble shifts and masks of `word`.
    asm("" : "+v"(lo), "+v"(hi));
    uint32_t o[4];
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const f32x2_t f = {fmaf((float)((lo >> (8 * p)) & 0xFFu), sc, bi),
                           fmaf((float)((hi >> (8 * p)) & 0xFFu), sc, bi)};
        o[p] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
    }
    return __builtin_bit_cast(bf16x8_t, make_uint4(o[0], o[1], o[2], o[3]));
}

// One K step of one thread's staging work, held in registers between the
// global loads and the LDS stores. X: the tile's 256 rows x 8 chunks of 16 bytes
// are numbered c = 8 * row + chunk and thread t loads chunks t, t + 512, ...,
// so 8 consecutive lanes read one row's 128 contiguous bytes (whole cache lines
// per instruction). W: the tile's 128 rows x 4 quarters of 8 bytes (2 words =
// 16 codes); thread t takes quarter t & 3 of row t >> 2 with its group's scale
// and bias.
template <bool XF32>
struct Stage {
    static constexpr int XCHUNKS = 4;                     // 16-byte bf16 chunks of X
    static constexpr int XLOADS = XCHUNKS * (XF32 ? 2 : 1);
    uint4 x[XLOADS];
    uint2 w;
    uint32_t s, b;  // raw scale / bias bits
};

constexpr int BM = 256, BN = 128, NT = 512;
constexpr int TILE_BYTES = (BM + BN) * ROW_BYTES;  // X tile + W tile of one step (48 KiB)

// All loads go through buffer resources (X rows past M and W rows past N read
// as zero), so this function has no branches and its loads stay in flight
// until the stage is stored.
template <bool XF32, int SBT>
__device__ __forceinline__ void load_stage(Stage<XF32>& st, __amdgpu_buffer_rsrc_t rx,
                                           __amdgpu_buffer_rsrc_t rw, __amdgpu_buffer_rsrc_t rs,
                                           __amdgpu_buffer_rsrc_t rb, uint32_t m0, uint32_t n0,
                                           uint32_t K, uint32_t P, uint32_t G, uint32_t k0, int gs_log2,
                                           int tid) {
    constexpr uint32_t XB = XF32 ? 4 : 2;
#pragma unroll
    for (int j = 0; j < Stage<XF32>::XCHUNKS; j++) {
        const uint32_t c = NT * j + tid;
        const uint32_t off = ((m0 + (c >> 3)) * K + k0 + 8 * (c & 7)) * XB;
        if constexpr (XF32) {
            const u32x4_t a = __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0);
            const u32x4_t b = __builtin_amdgcn_raw_buffer_load_b128(rx, off + 16, 0, 0);
            st.x[2 * j] = make_uint4(a.x, a.y, a.z, a.w);
            st.x[2 * j + 1] = make_uint4(b.x, b.y, b.z, b.w);
        } else {
            const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0);
            st.x[j] = make_uint4(v.x, v.y, v.z, v.w);
        }
    }
    const uint32_t n = n0 + (tid >> 2), qtr = tid & 3;
    typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
    const u32x2_t w = __builtin_amdgcn_raw_buffer_load_b64(rw, (n * P + (k0 >> 3) + 2 * qtr) * 4, 0, kAuxNT);
    st.w = make_uint2(w.x, w.y);
    const uint32_t g = (k0 + 16 * qtr) >> gs_log2;
    st.s = load_sb_bits<SBT>(rs, n * G + g);
    st.b = load_sb_bits<SBT>(rb, n * G + g);
}

// X chunk j of the stage into the LDS tile.
template <bool XF32>
__device__ __forceinline__ void store_x(const Stage<XF32>& st, uint8_t* buf, int tid, int j) {
    const int c = NT * j + tid;
    uint4 v;
    if constexpr (XF32) {
        const uint4 a = st.x[2 * j], b = st.x[2 * j + 1];
        v = make_uint4(pack_bf16x2(__uint_as_float(a.x), __uint_as_float(a.y)),
                       pack_bf16x2(__uint_as_float(a.z), __uint_as_float(a.w)),
                       pack_bf16x2(__uint_as_float(b.x), __uint_as_float(b.y)),
                       pack_bf16x2(__uint_as_float(b.z), __uint_as_float(b.w)));
    } else {
        v = st.x[j];
    }
    *reinterpret_cast<uint4*>(buf + swz(c >> 3, c & 7)) = v;
}

// Word j (0 or 1) of the thread's W quarter, dequantized to 8 bf16 in LDS.
__device__ __forceinline__ void store_w(uint32_t word, float sc, float bi, uint8_t* buf, int tid, int j) {
    uint8_t* ws = buf + BM * ROW_BYTES;
    const int row = tid >> 2, chunk = 2 * (tid & 3) + j;
    *reinterpret_cast<bf16x8_t*>(ws + swz(row, chunk)) = dequant_word(word, sc, bi);
}

template <bool XF32, int SBT>
__device__ __forceinline__ void store_stage(const Stage<XF32>& st, uint8_t* buf, int tid) {
#pragma unroll
    for (int j = 0; j < Stage<XF32>::XCHUNKS; j++) store_x<XF32>(st, buf, tid, j);
    const float sc = widen_sb<SBT>(st.s), bi = widen_sb<SBT>(st.b);
    store_w(st.w.x, sc, bi, buf, tid, 0);
    store_w(st.w.y, sc, bi, buf, tid, 1);
}

// 256 x 128 tile of Y per block of 8 waves (4 x 2), each wave 64 x 64 as 2 x 2
// 32x32 MFMA tiles. Each dequantized W element feeds 256 rows of X, and every
// thread dequantizes 16 codes per step, so the dequant's VALU work stays below
// the MFMA time; LDS (2 x 48 KiB) leaves room for one block of 8 waves per CU.
// Floats between the split-K partial slices of an M x N product (a multiple of
// 4, so every slice starts 16-byte aligned).
__host__ __device__ inline size_t split_stride(uint32_t M, uint32_t N) { return ((size_t)M * N + 3) & ~(size_t)3; }

template <bool SPLIT, bool XF32, int SBT>
__global__ __launch_bounds__(NT, 1) void qmm_mfma_kernel(
    const uint32_t* __restrict__ W, const void* __restrict__ S, const void* __restrict__ B,
    const void* __restrict__ X, void* __restrict__ Y, int y_dt, uint32_t M, uint32_t N, uint32_t K,
    int gs_log2, uint32_t k_per_split, float* __restrict__ acc_out) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * TILE_BYTES];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int wm = wave >> 1, wn = wave & 1;  // 4 x 2 waves
    const uint32_t P = K >> 3, G = K >> gs_log2;
    constexpr uint32_t sb_bytes = SBT == 2 ? 4 : 2;
    const auto rx = make_rsrc(X, M * K * (XF32 ? 4 : 2));
    const auto rw = make_rsrc(W, N * P * 4);
    const auto rs = make_rsrc(S, N * G * sb_bytes);
    const auto rb = make_rsrc(B, N * G * sb_bytes);
    const uint32_t kb = blockIdx.z * k_per_split;
    const uint32_t ke = min(K, kb + k_per_split);
    const int nsteps = kb < ke ? (int)((ke - kb) / BK) : 0;

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    // Two register stages: the loads of step s+2 are issued while step s is
    // multiplied, and step s+1 (loaded one step earlier) is dequantized into
    // the other LDS buffer between the MFMAs of step s.
    Stage<XF32> st0, st1;
    auto load = [&](Stage<XF32>& st, int step) {
        load_stage<XF32, SBT>(st, rx, rw, rs, rb, m0, n0, K, P, G, kb + (uint32_t)step * BK, gs_log2, tid);
    };
    auto mma = [&](const uint8_t* cur, const Stage<XF32>& nst, bool store_next, uint8_t* nxt) {
        const uint8_t* xs = cur;
        const uint8_t* ws = cur + BM * ROW_BYTES;
        bf16x8_t a[2][2], bb[2][2];
        auto frags = [&](int kk, int buf) {
            const int c = 2 * kk + (lane >> 5);
#pragma unroll
            for (int i = 0; i < 2; i++)
                a[buf][i] = *reinterpret_cast<const bf16x8_t*>(xs + swz(wm * 64 + 32 * i + (lane & 31), c));
#pragma unroll
            for (int j = 0; j < 2; j++)
                bb[buf][j] = *reinterpret_cast<const bf16x8_t*>(ws + swz(wn * 64 + 32 * j + (lane & 31), c));
        };
        float sc = 0.0f, bi = 0.0f;
        if (store_next) {
            sc = widen_sb<SBT>(nst.s);
            bi = widen_sb<SBT>(nst.b);
        }
        frags(0, 0);
#pragma unroll
        for (int kk = 0; kk < BK / 16; kk++) {
            if (kk + 1 < BK / 16) frags(kk + 1, (kk + 1) & 1);
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[kk & 1][i], bb[kk & 1][j], acc[i][j], 0, 0, 0);
            if (store_next) {
                store_x<XF32>(nst, nxt, tid, kk);
                if (kk < 2) store_w(kk == 0 ? nst.w.x : nst.w.y, sc, bi, nxt, tid, kk);
            }
        }
    };
    if (nsteps > 0) {
        load(st0, 0);
        if (nsteps > 1) load(st1, 1);
        store_stage<XF32, SBT>(st0, lds, tid);
    }
    __syncthreads();

    // invariant at the top of step s: LDS[s % 2] holds step s, the register
    // stage for step s+1 is in flight, the other register stage is free
    for (int s = 0; s < nsteps; s += 2) {
        if (s + 2 < nsteps) load(st0, s + 2);
        mma(lds, st1, s + 1 < nsteps, lds + TILE_BYTES);
        __syncthreads();
        if (s + 1 >= nsteps) break;
        if (s + 3 < nsteps) load(st1, s + 3);
        mma(lds + TILE_BYTES, st0, s + 2 < nsteps, lds);
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint32_t n = n0 + wn * 64 + 32 * j + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const uint32_t m = m0 + wm * 64 + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < M && n < N) {
                    if constexpr (SPLIT)
                        acc_out[blockIdx.z * split_stride(M, N) + (size_t)m * N + n] = acc[i][j][r];
                    else
                        store_y(Y, (int64_t)m * N + n, acc[i][j][r], y_dt);
                }
            }
        }
}

// y = the sum of the `split` partial products in ws (each M x N fp32, slices
// split_stride apart), added in split order: the result does not depend on
// which block ran first. Four elements per thread (16-byte loads), then a
// scalar tail.
__global__ void split_sum_kernel(const float* __restrict__ ws, int split, int64_t n, void* __restrict__ y,
                                 int y_dt) {
    const int64_t n4 = n >> 2;
    const size_t ss = (size_t)(n + 3) & ~(size_t)3;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
        float4 a = reinterpret_cast<const float4*>(ws)[i];
        for (int s = 1; s < split; s++) {
            const float4 b = reinterpret_cast<const float4*>(ws + s * ss)[i];
            a.x += b.x, a.y += b.y, a.z += b.z, a.w += b.w;
        }
        if (y_dt == JH_F32) {
            reinterpret_cast<float4*>(y)[i] = a;
        } else {
            const uint32_t lo = (uint32_t)f32_to_bf16_hw(a.x) | ((uint32_t)f32_to_bf16_hw(a.y) << 16);
            const uint32_t hi = (uint32_t)f32_to_bf16_hw(a.z) | ((uint32_t)f32_to_bf16_hw(a.w) << 16);
            reinterpret_cast<uint2*>(y)[i] = make_uint2(lo, hi);
        }
    }
    for (int64_t i = 4 * n4 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        float a = ws[i];
        for (int s = 1; s < split; s++) a += ws[s * ss + i];
        store_y(y, i, a, y_dt);
    }
}

int log2_exact(int v) {
    int l = 0;
    while ((1 << l) < v) l++;
    return ((1 << l) == v) ? l : -1;
}

// ---- W-in-registers tile ---------------------------------------------------------
//
// Lane l of v_mfma_f32_32x32x16_bf16 supplies B[k = 8*(l/32) .. +8][j = l % 32]:
// eight consecutive k of one weight row, i.e. exactly one packed word. So W
// never goes through LDS: each wave loads its columns' words straight into
// registers and dequantizes them into B fragments just before the MFMAs that
// use them; only X is staged in LDS, shared by every wave of the block.
//
// K is walked in super-steps of 256 (four 64-wide steps). Inside a super-step
// the K order is permuted identically on both operands so that every lane's
// weights are one contiguous 64-byte run of its row: lane half h holds words
// 16h .. 16h+15 of the row's 128-byte super-step segment, and MFMA k16 step s of
// step t uses word 16h + 4t + s, i.e. actual k = 128h + 32t + 8s .. +8. The X tile
// of step t therefore holds, per row, the k runs [32t, 32t+32) and
// [128+32t, 128+32t+32) as logical 16-byte chunks 0-3 and 4-7, and lane half h
// reads chunk 4h + s. A lane's scales and biases for a super-step are
// 128/group_size consecutive groups, fetched with one load each.
//
// Each wave owns a 128 x (32*WNF) block of Y (4 x WNF MFMA tiles), so every
// dequantized weight feeds 128 rows of X.
constexpr int RBM = 128;                    // rows of X per block (and per wave)
constexpr int RXT = RBM * ROW_BYTES;        // 16 KiB X tile per K step

// Scales/biases of one lane for one super-step of SUP: the lane's K half spans
// SUP/2 elements, i.e. NG groups (at least one).
template <int SBT, int GSL, int SUP>
struct SbRegs {
    static constexpr int NG = ((SUP / 2) >> GSL) > 0 ? ((SUP / 2) >> GSL) : 1;
    static constexpr int BYTES = NG * (SBT == 2 ? 4 : 2);
    static constexpr int WORDS = BYTES >= 4 ? BYTES / 4 : 1;
    uint32_t s[WORDS], b[WORDS];
};

template <int SBT, int GSL, int SUP>
__device__ __forceinline__ void load_sb_run(SbRegs<SBT, GSL, SUP>& r, __amdgpu_buffer_rsrc_t rs,
                                            __amdgpu_buffer_rsrc_t rb, uint32_t off) {
    using R = SbRegs<SBT, GSL, SUP>;
    if constexpr (R::BYTES == 2) {
        r.s[0] = buf_load2(rs, off);
        r.b[0] = buf_load2(rb, off);
    } else if constexpr (R::BYTES == 4) {
        r.s[0] = __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0);
        r.b[0] = __builtin_amdgcn_raw_buffer_load_b32(rb, off, 0, 0);
    } else if constexpr (R::BYTES == 8) {
        typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
        const u32x2_t a = __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, 0);
        const u32x2_t c = __builtin_amdgcn_raw_buffer_load_b64(rb, off, 0, 0);
        r.s[0] = a.x, r.s[1] = a.y, r.b[0] = c.x, r.b[1] = c.y;
    } else {
        const u32x4_t a = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
        const u32x4_t c = __builtin_amdgcn_raw_buffer_load_b128(rb, off, 0, 0);
        r.s[0] = a.x, r.s[1] = a.y, r.s[2] = a.z, r.s[3] = a.w;
        r.b[0] = c.x, r.b[1] = c.y, r.b[2] = c.z, r.b[3] = c.w;
    }
}

// Group element e of a lane's run as fp32.
template <int SBT, int GSL>
__device__ __forceinline__ float sb_elem(const uint32_t* words, int e) {
    if constexpr (SBT == 2) return __uint_as_float(words[e]);
    const uint32_t w = words[e >> 1];
    const uint16_t h16 = (e & 1) ? (uint16_t)(w >> 16) : (uint16_t)w;
    return SBT == 1 ? f16_to_f32(h16) : bf16_to_f32(h16);
}

template <int WNF, int SBT, int GSL, int SUP>
struct WRegs {
    uint4 w[WNF][SUP / 64];     // SUP/16 words of column j for this lane's K half
    SbRegs<SBT, GSL, SUP> sb[WNF];
};

// Physical 16-byte chunk of logical chunk c in row r of an X tile.
__device__ __forceinline__ uint32_t xswz(int r, int c) { return r * ROW_BYTES + ((c ^ ((r >> 1) & 7)) << 4); }

template <bool SPLIT, bool XF32, int SBT, int GSL, int NW, int WNF, int SUP>
__global__ __launch_bounds__(64 * NW, 2) void qmm_wreg_kernel(
    const uint32_t* __restrict__ W, const void* __restrict__ S, const void* __restrict__ B,
    const void* __restrict__ X, void* __restrict__ Y, int y_dt, uint32_t M, uint32_t N, uint32_t K,
    uint32_t k_per_split, float* __restrict__ acc_out) {
    constexpr int NTH = 64 * NW;
    constexpr int RBN = 32 * WNF * NW;
    constexpr int XCH = (RBM * 8 + NTH - 1) / NTH;  // 16-byte X chunks per thread per step
    constexpr bool XPART = RBM * 8 % NTH != 0;        // 6 waves: the last chunk is held by part of the block
    constexpr int XL = XCH * (XF32 ? 2 : 1);
    constexpr uint32_t SBB = SBT == 2 ? 4 : 2;
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * RXT];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = lane >> 5, c32 = lane & 31;
    const uint32_t m0 = blockIdx.y * RBM, n0 = blockIdx.x * RBN + wave * 32 * WNF;
    const uint32_t P = K >> 3, G = K >> GSL;
    const auto rx = make_rsrc(X, M * K * (XF32 ? 4 : 2));
    const auto rw = make_rsrc(W, N * P * 4);
    const auto rs = make_rsrc(S, N * G * SBB);
    const auto rb = make_rsrc(B, N * G * SBB);
    const uint32_t kb = blockIdx.z * k_per_split;
    const uint32_t ke = min(K, kb + k_per_split);
    constexpr int SPS = SUP / 64;  // 64-wide steps per super-step
    const int nsup = kb < ke ? (int)((ke - kb) / SUP) : 0;  // super-steps
    const int nsteps = SPS * nsup;

    floatx16 acc[4][WNF];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < WNF; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    // Super-steps past the last are clamped to it: their loads are repeats, so
    // the pipeline needs no branches.
    auto ksup = [&](int sup) { return kb + (uint32_t)min(sup, nsup - 1) * SUP; };
    auto load_w = [&](WRegs<WNF, SBT, GSL, SUP>& wr, int sup) {
        const uint32_t k0 = ksup(sup);
        const uint32_t g0 = (k0 + (SUP / 2) * h) >> GSL;
#pragma unroll
        for (int j = 0; j < WNF; j++) {
            const uint32_t n = n0 + 32 * j + c32;
            const uint32_t off = (n * P + (k0 >> 3) + (SUP / 16) * h) * 4;
#pragma unroll
            for (int q = 0; q < SPS; q++) wr.w[j][q] = buf_load16_nt(rw, off + 16 * q);
            load_sb_run<SBT, GSL, SUP>(wr.sb[j], rs, rb, (n * G + g0) * SBB);
        }
    };
    struct XRegs {
        uint4 v[XL];
    };
    // X of step `step` (super-step step/SPS, t = step%SPS): logical chunk c of
    // row r holds k = (SUP/2)*(c/4) + 32t + 8*(c%4) .. +8 of the super-step.
    auto load_x = [&](XRegs& xr, int step) {
        const uint32_t k0 = ksup(step / SPS) + 32 * (step % SPS);
#pragma unroll
        for (int q = 0; q < XCH; q++) {
            const uint32_t c0 = NTH * q + tid;
            const uint32_t c = XPART && c0 >= RBM * 8 ? 0 : c0;  // past the tile: a repeat of chunk 0, never stored
            const uint32_t kc = k0 + (SUP / 2) * ((c >> 2) & 1) + 8 * (c & 3);
            const uint32_t off = ((m0 + (c >> 3)) * K + kc) * (XF32 ? 4 : 2);
            if constexpr (XF32) {
                const u32x4_t a = __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0);
                const u32x4_t b = __builtin_amdgcn_raw_buffer_load_b128(rx, off + 16, 0, 0);
                xr.v[2 * q] = make_uint4(a.x, a.y, a.z, a.w);
                xr.v[2 * q + 1] = make_uint4(b.x, b.y, b.z, b.w);
            } else {
                const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0);
                xr.v[q] = make_uint4(v.x, v.y, v.z, v.w);
            }
        }
    };
    auto store_xq = [&](const XRegs& xr, uint8_t* buf, int q) {
        const int c = NTH * q + tid;
        if (XPART && c >= RBM * 8) return;
        uint4 v;
        if constexpr (XF32) {
            const uint4 a = xr.v[2 * q], b = xr.v[2 * q + 1];
            v = make_uint4(pack_bf16x2(__uint_as_float(a.x), __uint_as_float(a.y)),
                           pack_bf16x2(__uint_as_float(a.z), __uint_as_float(a.w)),
                           pack_bf16x2(__uint_as_float(b.x), __uint_as_float(b.y)),
                           pack_bf16x2(__uint_as_float(b.z), __uint_as_float(b.w)));
        } else {
            v = xr.v[q];
        }
        *reinterpret_cast<uint4*>(buf + xswz(c >> 3, c & 7)) = v;
    };

    // Step t of a super-step: X from LDS `xs`, W words 4t..4t+3 of `wr`; the X
    // chunks of the next step (in xr) are stored into `xn` between the MFMAs.
    // The A fragments and B fragments of k16 step s+1 are produced while the
    // MFMAs of step s run.
    auto compute = [&](const uint8_t* xs, const WRegs<WNF, SBT, GSL, SUP>& wr, int t, const XRegs& xr,
                       uint8_t* xn, bool live) {
        float sc[WNF], bi[WNF];
#pragma unroll
        for (int j = 0; j < WNF; j++) {
            const int e = (32 * t) >> GSL;  // group of this step inside the lane's run
            sc[j] = sb_elem<SBT, GSL>(wr.sb[j].s, e);
            bi[j] = sb_elem<SBT, GSL>(wr.sb[j].b, e);
        }
        bf16x8_t a[2][4], bq[2][WNF];
        auto read_a = [&](int s, int buf) {
#pragma unroll
            for (int i = 0; i < 4; i++)
                a[buf][i] = *reinterpret_cast<const bf16x8_t*>(xs + xswz(32 * i + c32, 4 * h + s));
        };
        auto deq = [&](int s, int buf) {
#pragma unroll
            for (int j = 0; j < WNF; j++) {
                const uint4 q4 = wr.w[j][t];
                const uint32_t word = s == 0 ? q4.x : s == 1 ? q4.y : s == 2 ? q4.z : q4.w;
                bq[buf][j] = dequant_word(word, sc[j], bi[j]);
            }
        };
        read_a(0, 0);
        deq(0, 0);
#pragma unroll
        for (int s = 0; s < 4; s++) {
            if (s < 3) {
                read_a(s + 1, (s + 1) & 1);
                deq(s + 1, (s + 1) & 1);
            }
            if (live) {
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int j = 0; j < WNF; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[s & 1][i], bq[s & 1][j], acc[i][j], 0, 0, 0);
            }
            if (s < XCH) store_xq(xr, xn, s);
        }
#pragma unroll
        for (int q = 4; q < XCH; q++) store_xq(xr, xn, q);
    };

    // W: two super-step slots (the next super-step's runs load during the
    // current one). X: two register sets, about one and a half steps ahead, and
    // two LDS buffers (step t+1 is stored during step t).
    WRegs<WNF, SBT, GSL, SUP> wa, wb;
    XRegs xa, xb;
    if (nsteps > 0) {
        load_x(xa, 0);
        load_w(wa, 0);
        load_x(xb, 1);
#pragma unroll
        for (int q = 0; q < XCH; q++) store_xq(xa, lds, q);
        load_x(xa, 2);
    }
    __syncthreads();
    // top of step t: LDS[t % 2] holds X of step t; X of steps t+1 and t+2 are in
    // the register sets (t+1) % 2 and t % 2.
    auto step = [&](int t, WRegs<WNF, SBT, GSL, SUP>& wcur, XRegs& xnext, uint8_t* lcur, uint8_t* lnext) {
        compute(lcur, wcur, t % SPS, xnext, lnext, t < nsteps);
        load_x(xnext, t + 3);
        __syncthreads();
    };
    // Unrolled over two super-steps (the W slots) with no early exit: an exit
    // per step would keep one copy of the accumulators live per exit. Steps past
    // the end skip their MFMAs. SPS is even, so step parity (LDS buffer and X
    // register set) is static.
    for (int t = 0; t < nsteps; t += 2 * SPS) {
        load_w(wb, t / SPS + 1);
#pragma unroll
        for (int u = 0; u < SPS; u += 2) {
            step(t + u, wa, xb, lds, lds + RXT);
            step(t + u + 1, wa, xa, lds + RXT, lds);
        }
        load_w(wa, t / SPS + 2);
#pragma unroll
        for (int u = 0; u < SPS; u += 2) {
            step(t + SPS + u, wb, xb, lds, lds + RXT);
            step(t + SPS + u + 1, wb, xa, lds + RXT, lds);
        }
    }

#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < WNF; j++) {
            const uint32_t n = n0 + 32 * j + c32;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const uint32_t m = m0 + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
                if (m < M && n < N) {
                    if constexpr (SPLIT)
                        acc_out[blockIdx.z * split_stride(M, N) + (size_t)m * N + n] = acc[i][j][r];
                    else
                        store_y(Y, (int64_t)m * N + n, acc[i][j][r], y_dt);
                }
            }
        }
}


// ---- The same tile with its operands staged in LDS rings ---------------------------
//
// Every load of a step — the X tile, the wave's 16 bytes of weight words per lane
// and, once per super-step, its scales and biases — is a buffer load with an LDS
// destination, issued A steps before the step that reads it. Nothing in flight
// holds registers, so the loads get A steps (A+1 LDS slots) to land, where the
// register tile's weights had about two; and the X tile needs no register
// staging or LDS stores. The LDS layout, the K permutation, the dequantization
// and the MFMA order are those of qmm_wreg_kernel, so the two tiles give the
// same bits.
//
// The loads are issued from inline asm with explicit waits: the compiler tracks
// loads into LDS it issued itself and makes each LDS read wait for all of them
// (vmcnt(0)), which would drain the ring every step. Loads complete in issue
// order, so at the top of step t `s_waitcnt vmcnt(n)` with n = the loads issued
// after step t's own leaves exactly those in flight; any load the compiler adds
// in between only makes the wait longer, never shorter.

// LDS byte offset of a __shared__ address (the value M0 takes for a load into LDS).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return __builtin_amdgcn_readfirstlane((uint32_t)(size_t)(__attribute__((address_space(3))) const void*)p);
}
// 16 bytes per lane into LDS at m0 + 16 * lane (the s_nop covers the M0 write).
__device__ __forceinline__ void lds_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t m0) {
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(r), "{m0}"(m0) : "memory");
}
// The same with a wave-uniform part of the offset in soff; the range check
// applies to voff, which carries the row, so rows past the buffer still read 0.
__device__ __forceinline__ void lds_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, uint32_t m0) {
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(r),
                 "s"(__builtin_amdgcn_readfirstlane(soff)), "{m0}"(m0)
                 : "memory");
}
// 4 bytes per lane into LDS at m0 + 4 * lane.
__device__ __forceinline__ void lds_load4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t m0) {
    asm volatile("s_nop 0\n\tbuffer_load_dword %0, %1, 0 offen lds" ::"v"(voff), "s"(r), "{m0}"(m0) : "memory");
}
template <int N>
__device__ __forceinline__ void wait_vmem() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Dwords of scales (and of biases) per lane per super-step: SUP/2 elements of
// the lane's K half are NG groups; 0 when they do not fill whole dwords.
template <int SBT, int GSL>
constexpr int dma_sb_dwords() {
    constexpr int ng = (128 >> GSL) > 0 ? (128 >> GSL) : 1;
    constexpr int bytes = ng * (SBT == 2 ? 4 : 2);
    return bytes % 4 == 0 ? bytes / 4 : 0;
}

// Loads a wave issues after those of step t (t % SPS = u): they were issued at
// step t - A, and steps t - A + v (v = 1 .. A-1) issue the loads of step t + v:
// NX X loads, and when t + v starts a super-step its 4 weight loads and 2·NSB
// scale/bias loads. (Step t's own weights and scales were issued no later than
// its X.)
template <int A, int NX, int NSB, int SPS>
constexpr int dma_loads_after(int u) {
    int n = 0;
    for (int v = 1; v < A; v++) n += NX + (((u + v) % SPS) == 0 ? 4 + 2 * NSB : 0);
    return n;
}

// The split-K partial tiles added inside the product's launch (INL): the S
// blocks of one output tile (blockIdx.z = 0 .. S-1) run on one XCD (the grid's
// x·y is a multiple of 8 and the GPU deals blocks to its 8 XCDs round-robin)
// and all blocks of the grid are resident at once (at most one per CU). Each
// stores its partial tile, counts its arrival in the tile's counter in the
// XCD's L2, waits until all S have arrived, then adds rows z·RB/S .. of the S
// partials (device-coherent loads from the L2) in split order -- the summing
// launch's order, so the same bits -- and stores them into Y. A second count
// per block tells the last one to reset the counter for the next call. The
// wait is bounded: a block that gives up stores NaN for its rows and sets the
// status word the library reports at the next synchronisation.
template <int S, int RB, int RBN, int NT>
__device__ __forceinline__ void split_tile_sum(const float* acc_out, size_t ss, void* Y, int y_dt, uint32_t M,
                                               uint32_t N, uint32_t mb, uint32_t nb, bool gave_up) {
    constexpr int C4 = RBN / 4, Q = RB / (8 * S);  // float4 items per thread
    static_assert(Q >= 1 && (RB / S) * C4 == Q * NT, "rows per share x columns / threads");
    const auto rp = make_rsrc(acc_out, (uint32_t)(S * ss * 4));
    const int tid = threadIdx.x;
    u32x4_t v[Q][S];
#pragma unroll
    for (int q = 0; q < Q; q++) {
        const int idx = tid + NT * q;
        const uint32_t m = mb + idx / C4, n = nb + 4 * (idx % C4);
        const bool in = m < M && n < N;
#pragma unroll
        for (int s = 0; s < S; s++)
            v[q][s] = in ? __builtin_amdgcn_raw_buffer_load_b128(rp, (uint32_t)((s * ss + (size_t)m * N + n) * 4), 0,
                                                                 kAuxSc1)
                         : u32x4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int q = 0; q < Q; q++) {
        const int idx = tid + NT * q;
        const uint32_t m = mb + idx / C4, n = nb + 4 * (idx % C4);
        if (m >= M || n >= N) continue;
        float4 a = make_float4(__uint_as_float(v[q][0].x), __uint_as_float(v[q][0].y), __uint_as_float(v[q][0].z),
                               __uint_as_float(v[q][0].w));
#pragma unroll
        for (int s = 1; s < S; s++) {
            a.x += __uint_as_float(v[q][s].x), a.y += __uint_as_float(v[q][s].y);
            a.z += __uint_as_float(v[q][s].z), a.w += __uint_as_float(v[q][s].w);
        }
        if (gave_up) a = make_float4(__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""));
        const size_t o = (size_t)m * N + n;
        if (y_dt == JH_F32) {
            *reinterpret_cast<float4*>(static_cast<float*>(Y) + o) = a;
        } else {
            const uint32_t lo = (uint32_t)f32_to_bf16_hw(a.x) | ((uint32_t)f32_to_bf16_hw(a.y) << 16);
            const uint32_t hi = (uint32_t)f32_to_bf16_hw(a.z) | ((uint32_t)f32_to_bf16_hw(a.w) << 16);
            *reinterpret_cast<uint2*>(static_cast<uint16_t*>(Y) + o) = make_uint2(lo, hi);
        }
    }
}

template <bool SPLIT, int SBT, int GSL, int NW, int A, int RB = RBM, bool INL = false>  // RB: rows of X per block, 32 | 64 | 128 | 256
__global__ __launch_bounds__(64 * NW, RB == 256 ? 1 : 2) void qmm_dma_kernel(
    const uint32_t* __restrict__ W, const void* __restrict__ S, const void* __restrict__ B,
    const void* __restrict__ X, void* __restrict__ Y, int y_dt, uint32_t M, uint32_t N, uint32_t K,
    uint32_t k_per_split, float* __restrict__ acc_out, InLaunchSync sy) {
    constexpr int SUP = 256, SPS = SUP / 64, R = A + 1;
    static_assert(A >= 1 && A <= SPS, "the scale/bias ring has two super-step slots");
    constexpr int RBN = 32 * NW;
    constexpr uint32_t SBB = SBT == 2 ? 4 : 2;
    constexpr int NSB = dma_sb_dwords<SBT, GSL>();
    static_assert(NSB >= 1, "scales/biases in whole dwords");
    static_assert(RB == 32 || RB == 64 || RB == 128 || RB == 256, "rows per block");
    constexpr int RT = RB / 32;                 // MFMA row tiles per wave
    constexpr int XT = RB * ROW_BYTES;          // X tile per K step
    constexpr int XQ = XT / 1024;               // 1 KiB loads per X tile (8 rows each)
    constexpr int NX = (XQ + NW - 1) / NW;      // X loads per wave per step
    constexpr int WSLOT = NW * 4096;            // weight words of one super-step, all waves
    constexpr int SBW = 2 * NSB * 256;          // one wave's scales + biases of a super-step
    constexpr int JUNK = NX * NW > XQ ? 1024 : 0;  // target of the filler loads that even out the count
    __shared__ __attribute__((aligned(16))) uint8_t lds[R * XT + 2 * WSLOT + 2 * NW * SBW + JUNK];
    uint8_t* const xring = lds;
    uint8_t* const wring = lds + R * XT;  // two super-step slots
    uint8_t* const sbring = wring + 2 * WSLOT;
    uint8_t* const junk = sbring + 2 * NW * SBW;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, c32 = lane & 31;
    const uint32_t m0 = blockIdx.y * RB, n0 = blockIdx.x * RBN + wave * 32;
    const uint32_t P = K >> 3, G = K >> GSL;
    const auto rx = make_rsrc(X, M * K * 2);
    const auto rw = make_rsrc(W, N * P * 4);
    const auto rs = make_rsrc(S, N * G * SBB);
    const auto rb = make_rsrc(B, N * G * SBB);
    const uint32_t kb = blockIdx.z * k_per_split;
    const uint32_t ke = min(K, kb + k_per_split);
    const int nsup = kb < ke ? (int)((ke - kb) / SUP) : 0;
    const int nsteps = SPS * nsup;

    floatx16 acc[RT];
#pragma unroll
    for (int i = 0; i < RT; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[i][r] = 0.0f;

    // Super-steps past the last are clamped to it: their loads are repeats into
    // slots nobody reads, so every step issues the same number of loads.
    auto ksup = [&](int sup) { return kb + (uint32_t)min(sup, nsup - 1) * SUP; };
    // The loads of step s into ring slot s % R.
    auto issue = [&](int s) {
        const int slot = s % R, t = s % SPS;
        const uint32_t k0 = ksup(s / SPS);
        // X: load q is rows 8q .. 8q+7 of the tile; lane -> (row, physical chunk p)
        // holding logical chunk p ^ ((row/2) % 8) (the swizzle is applied on the source side)
#pragma unroll
        for (int i = 0; i < NX; i++) {
            const int q = wave + NW * i;
            const int qs = q < XQ ? q : q - XQ;  // a filler repeats a real load into junk
            const int r = 8 * qs + (lane >> 3), c = (lane & 7) ^ ((r >> 1) & 7);
            const uint32_t kc = (SUP / 2) * (c >> 2) + 8 * (c & 3);
            lds_load16(rx, ((m0 + r) * K + kc) * 2, (k0 + 32 * t) * 2,
                       lds_addr(q < XQ ? xring + slot * XT + 1024 * q : junk));
        }
        if (t == 0) {  // the super-step's weights, scales and biases
            // weights: the 128-byte super-step segments of the wave's 32 columns as
            // whole lines, load i holding rows 8i .. 8i+7; 16-byte chunk c of row r
            // sits at position c ^ ((r/2) % 8), so that the step's reads (chunk
            // 4h + t of row c32 by lane (h, c32)) spread over the banks
            uint8_t* const wbase = wring + ((s / SPS) & 1) * WSLOT + 4096 * wave;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = 8 * i + (lane >> 3), c = (lane & 7) ^ ((r >> 1) & 7);
                lds_load16(rw, ((n0 + r) * P + 4 * c) * 4, (k0 >> 3) * 4, lds_addr(wbase + 1024 * i));
            }
            uint8_t* const base = sbring + (((s / SPS) & 1) * NW + wave) * SBW;
            const uint32_t off = ((n0 + c32) * G + ((k0 + (SUP / 2) * h) >> GSL)) * SBB;
#pragma unroll
            for (int i = 0; i < NSB; i++) lds_load4(rs, off + 4 * i, lds_addr(base + 256 * i));
#pragma unroll
            for (int i = 0; i < NSB; i++) lds_load4(rb, off + 4 * i, lds_addr(base + 256 * (NSB + i)));
        }
    };
    auto compute = [&](int s) {
        const int slot = s % R, t = s % SPS;
        const uint8_t* const xs = xring + slot * XT;
        const uint4 wq = *reinterpret_cast<const uint4*>(wring + ((s / SPS) & 1) * WSLOT + 4096 * wave + 128 * c32 +
                                                          16 * ((4 * h + t) ^ ((c32 >> 1) & 7)));
        const uint8_t* const sbb = sbring + (((s / SPS) & 1) * NW + wave) * SBW;
        uint32_t sw[NSB], bw[NSB];
#pragma unroll
        for (int i = 0; i < NSB; i++) {
            sw[i] = *reinterpret_cast<const uint32_t*>(sbb + 256 * i + 4 * lane);
            bw[i] = *reinterpret_cast<const uint32_t*>(sbb + 256 * (NSB + i) + 4 * lane);
        }
        const int e = (32 * t) >> GSL;
        const float sc = sb_elem<SBT, GSL>(sw, e), bi = sb_elem<SBT, GSL>(bw, e);
        bf16x8_t a[2][RT], bq[2];
        auto read_a = [&](int k, int buf) {
#pragma unroll
            for (int i = 0; i < RT; i++)
                a[buf][i] = *reinterpret_cast<const bf16x8_t*>(xs + xswz(32 * i + c32, 4 * h + k));
        };
        auto deq = [&](int k, int buf) {
            const uint32_t word = k == 0 ? wq.x : k == 1 ? wq.y : k == 2 ? wq.z : wq.w;
            bq[buf] = dequant_word(word, sc, bi);
        };
        read_a(0, 0);
        deq(0, 0);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            if (k < 3) {
                read_a(k + 1, (k + 1) & 1);
                deq(k + 1, (k + 1) & 1);
            }
#pragma unroll
            for (int i = 0; i < RT; i++)
                acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[k & 1][i], bq[k & 1], acc[i], 0, 0, 0);
        }
    };
    if (nsteps > 0) {
#pragma unroll
        for (int s = 0; s < A; s++) issue(s);
        auto step = [&](int t, auto uc) {
            constexpr int u = decltype(uc)::value;
            wait_vmem<dma_loads_after<A, NX, NSB, SPS>(u)>();  // this step's loads have landed (this wave's) ...
            __syncthreads();  // ... and every wave's; slot (t+u-1) % R is free
            issue(t + u + A);
            compute(t + u);
        };
        for (int t = 0; t < nsteps; t += SPS) {
            static_assert(SPS == 4, "four steps per super-step");
            step(t, std::integral_constant<int, 0>{});
            step(t, std::integral_constant<int, 1>{});
            step(t, std::integral_constant<int, 2>{});
            step(t, std::integral_constant<int, 3>{});
        }
        wait_vmem<0>();  // no load may still target LDS when the block ends
    }

#pragma unroll
    for (int i = 0; i < RT; i++) {
        const uint32_t n = n0 + c32;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const uint32_t m = m0 + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
            if (m < M && n < N) {
                if constexpr (SPLIT)
                    acc_out[blockIdx.z * split_stride(M, N) + (size_t)m * N + n] = acc[i][r];
                else
                    store_y(Y, (int64_t)m * N + n, acc[i][r], y_dt);
            }
        }
    }
    if constexpr (INL) {
        static_assert(SPLIT && RB <= 128, "in-launch sums of split tiles of up to 128 rows");
        // the block's partial stores are in the XCD's L2 (they write through the
        // CU's L1) before its arrival is counted
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        const int nsplit = (int)gridDim.z;
        int* const cnt = sy.counters + 32 * (blockIdx.x + gridDim.x * blockIdx.y);
        // the rings are idle now (every wave is past its last step and its loads
        // have landed): their first word carries the wait's outcome
        int& gave_up_s = *reinterpret_cast<int*>(lds);
        if (tid == 0) {
            __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            bool seen = false;
            for (uint32_t n = 0; n < sy.spin; n++)
                if (__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= nsplit) {
                    seen = true;
                    break;
                }
            if (!seen) __hip_atomic_store(sy.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            gave_up_s = !seen;
        }
        __syncthreads();
        const bool gave_up = gave_up_s != 0;
        const size_t ss = split_stride(M, N);
        const uint32_t nb = blockIdx.x * RBN;
        const uint32_t mb = blockIdx.y * RB + blockIdx.z * (uint32_t)(RB / nsplit);
        if (nsplit == 2) split_tile_sum<2, RB, RBN, 64 * NW>(acc_out, ss, Y, y_dt, M, N, mb, nb, gave_up);
        else if (nsplit == 4) split_tile_sum<4, RB, RBN, 64 * NW>(acc_out, ss, Y, y_dt, M, N, mb, nb, gave_up);
        else if constexpr (RB >= 64) split_tile_sum<8, RB, RBN, 64 * NW>(acc_out, ss, Y, y_dt, M, N, mb, nb, gave_up);
        // every thread's partial loads have returned (their sums are stored)
        __syncthreads();
        if (tid == 0 && __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 2 * nsplit - 1)
            __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

}  // namespace

Status launch_generic(const QuantMatrix& m, const void* x, int x_dtype, int64_t rows, void* y,
                      int y_dtype, int num_cus, hipStream_t st);

constexpr int kBM = BM, kBN = BN;  // the LDS tile

// How one prefill product is launched. K divisible by 256 takes a tile of
// 32·waves columns of Y per block with K split 1, 2, 4 or 8 ways; each K range
// stores its fp32 partial tile, and one pass sums them in order. With scales in
// whole dwords per lane, X (fp32 X rounded to bf16 first) takes the LDS-ring tile: up to 64 rows in
// 32- or 64-row blocks; beyond, 128-row blocks of 4 waves with a lead of 1 step
// (two blocks per CU) or 3 steps (one), or of 8 waves with a lead of 3, and
// from 256 rows also 256-row blocks of 8 waves with a lead of 1. Otherwise
// the 128-row register tile with 4, 6 or 8 waves. The plan is the one with the
// least modelled time: the busiest CU's blocks, each costing a fixed start plus
// its columns x K super-steps at the CU's measured rate for that shape, plus a
// fixed and a per-element cost of the split (partial stores, the summing
// pass). The constants are least-squares fits to timed plans of the Qwen3-8B
// projections (N x K = 12288/6144/4096 x 4096, 4096 x 12288) on MI355X: for the
// LDS-ring tile at M = 128 .. 2048 6.6 % rms over 532 plans, the fitted choices
// taking 2364 us summed over 32 cases against 2361 us for the best plan of each
// (2436 us without the 256-row blocks); at M = 9 .. 64 5.6 % rms, 250.7 against
// 244.9 us over 16 cases; for the register tile 4.8 % rms over 320 plans, 3079
// against 3075 us over 32 cases. Other K (multiples of 64) take the LDS tile.
struct QmmPlan {
    bool wreg;
    int nw;
    int lead;  // steps of lead of the LDS-ring tile; 0: the register tile
    int rb;    // rows of X per block (LDS-ring tile: 32 or 64 up to 64 rows, 128 or 256 beyond)
    int64_t split;
    bool inl;  // the split's partial tiles are added inside the launch
    uint32_t k_per_split;
    dim3 grid;
};

// Whether an LDS-ring plan's split partials can be added inside its launch:
// 128-row blocks, every block resident at once (at most one per CU), the S
// blocks of a tile on one XCD (x·y a multiple of 8), a counter per tile, each
// block's share a whole number of 4-column items per thread, and the partials
// within a buffer resource's 2 GiB.
bool qmm_inl_fits(int64_t M, int64_t N, int nw, int rb, int64_t split, int num_cus) {
    if (rb != 128 || split < 2 || split > 8 || N % 4 != 0) return false;
    const int64_t rbn = 32 * nw, tiles = ((N + rbn - 1) / rbn) * ((M + rb - 1) / rb);
    return tiles % 8 == 0 && tiles <= kQmmSyncTiles && tiles * split <= num_cus / 8 * 8 &&
           (size_t)split * split_stride((uint32_t)M, (uint32_t)N) * 4 < ((size_t)1 << 31);
}

// Modelled microseconds of one LDS-ring plan (see above).
double qmm_dma_cost(int64_t M, int64_t N, int64_t nsup, int nw, int lead, int rb, int64_t split, int num_cus) {
    // the summing launch: fixed µs and µs per 10^6 partial sums (each table's own fit)
    const double kSplitFixed = rb < 128 ? 4.51 : 3.71;
    const double kSplitElem = rb < 128 ? 1.075 : 1.017;
    const int64_t rbn = 32 * nw, mt = (M + rb - 1) / rb;
    const int64_t blocks = ((N + rbn - 1) / rbn) * mt * split;
    const int64_t per_cu = (blocks + num_cus - 1) / num_cus;
    const double u = (double)rbn * (double)((nsup + split - 1) / split);
    // two 4-wave blocks share a CU: pairs at the pair rate, a last odd block alone
    auto pairs = [&](double rate2, double rate1, double start) {
        return (double)(per_cu / 2) * (2.0 * u / rate2 + start) + (double)(per_cu % 2) * (u / rate1 + start);
    };
    double t;
    if (rb == 32)
        t = nw == 4 ? pairs(110.5, 104.2, 2.70) : (double)per_cu * (u / 124.9 + 2.60);
    else if (rb == 64)
        t = nw == 4 ? pairs(95.2, 82.2, 3.22) : (double)per_cu * (u / 106.2 + 2.99);
    else if (rb == 256)
        t = (double)per_cu * (u / 47.1 + 7.87);
    else if (nw == 4 && lead == 1)
        t = pairs(65.2, 51.3, 3.50);
    else if (nw == 4)
        t = (double)per_cu * (u / 57.7 + 3.28);
    else
        t = (double)per_cu * (u / 75.4 + 5.15);
    if (split > 1) t += kSplitFixed + kSplitElem * (double)(M * N * split) * 1e-6;
    return t;
}

// Modelled microseconds of one W-in-registers plan (see above).
double qmm_wreg_cost(int64_t M, int64_t N, int64_t nsup, int nw, int64_t split, int num_cus) {
    constexpr double kRate4 = 37.0;      // column·super-steps per µs, one 4-wave block on a CU
    constexpr double kRate4x2 = 44.0;    // two 4-wave blocks on a CU
    constexpr double kRate6 = 43.0;      // one 6-wave block
    constexpr double kRate8 = 49.9;      // one 8-wave block
    constexpr double kBlockStart = 3.9;  // µs per block (per pair of 4-wave blocks) a CU runs in turn
    constexpr double kSplitFixed = 5.9;  // µs: the summing launch
    constexpr double kSplitElem = 1.04;  // µs per 10^6 partial sums
    const int64_t rbn = 32 * nw, mt = (M + RBM - 1) / RBM;
    const int64_t blocks = ((N + rbn - 1) / rbn) * mt * split;
    const int64_t per_cu = (blocks + num_cus - 1) / num_cus;
    const double u = (double)rbn * (double)((nsup + split - 1) / split);
    double t;
    if (nw == 4)
        t = (double)(per_cu / 2) * (2.0 * u / kRate4x2 + kBlockStart) + (double)(per_cu % 2) * (u / kRate4 + kBlockStart);
    else
        t = (double)per_cu * (u / (nw == 6 ? kRate6 : kRate8) + kBlockStart);
    if (split > 1) t += kSplitFixed + kSplitElem * (double)(M * N * split) * 1e-6;
    return t;
}

QmmPlan qmm_plan(const QuantMatrix& m, int64_t rows, int num_cus, bool dma, bool inl_ok = false) {
    QmmPlan p{};
    if (m.in % 256 == 0) {
        p.wreg = true;
        const int64_t nsup = m.in / 256;
        double best = 0;
        p.rb = RBM;
        if (dma) {
            // waves, lead, rows per block: 32/64-row blocks up to 64 rows, 128-row
            // blocks beyond, and 256-row blocks from 256 rows (8 waves with a lead
            // of 2 were never the modelled best over the shapes the fit covers)
            static constexpr int kSmall[4][3] = {{4, 3, 32}, {8, 3, 32}, {4, 2, 64}, {8, 2, 64}};
            static constexpr int kShapes[4][3] = {{8, 3, 128}, {4, 3, 128}, {4, 1, 128}, {8, 1, 256}};
            const int(*tab)[3] = rows <= 64 ? kSmall : kShapes;
            const int nshapes = rows <= 64 ? 4 : rows >= 256 ? 4 : 3;
            for (int i = 0; i < nshapes; i++) {
                const int nw = tab[i][0], lead = tab[i][1], rb = tab[i][2];
                for (int64_t split = 1; split <= (nw == 4 ? 8 : 4) && (split == 1 || nsup / split >= 2); split *= 2) {
                    const double t = qmm_dma_cost(rows, m.rows, nsup, nw, lead, rb, split, num_cus);
                    if (p.nw == 0 || t < best) best = t, p.nw = nw, p.lead = lead, p.rb = rb, p.split = split;
                }
            }
            // a 4-wave plan's partials of a 4- or 8-way split are added inside its
            // launch where they can be: timed on MI355X against the summing launch
            // for the Qwen3-8B projections at M = 65 .. 512, 0.1 to 5.4 us faster for
            // every plan the model picks (o_proj at M = 128: 15.4 against 20.8 us);
            // 2-way splits came out within +-0.8 us and 8-wave blocks up to 3.7 us
            // slower, so they keep the summing launch
            p.inl = inl_ok && p.nw == 4 && p.split >= 4 && qmm_inl_fits(rows, m.rows, p.nw, p.rb, p.split, num_cus);
        } else {
            for (int nw : {8, 4, 6})
                for (int64_t split = 1; split <= (nw == 4 ? 8 : 4) && (split == 1 || nsup / split >= 2); split *= 2) {
                    const double t = qmm_wreg_cost(rows, m.rows, nsup, nw, split, num_cus);
                    if (p.nw == 0 || t < best) best = t, p.nw = nw, p.split = split;
                }
        }
        const int64_t rbn = 32 * p.nw;
        p.k_per_split = (uint32_t)(((nsup + p.split - 1) / p.split) * 256);
        p.grid = dim3((unsigned)((m.rows + rbn - 1) / rbn), (unsigned)((rows + p.rb - 1) / p.rb), (unsigned)p.split);
        return p;
    }
    p.wreg = false;
    p.nw = NT / 64;
    const int64_t tiles = ((m.rows + kBN - 1) / kBN) * ((rows + kBM - 1) / kBM);
    const int64_t ksteps = m.in / BK;
    p.split = 1;
    // aim for two tiles per CU, keep at least 8 K steps per split
    while (tiles * p.split < 2 * num_cus && ksteps / (p.split * 2) >= 8) p.split *= 2;
    p.k_per_split = (uint32_t)(((ksteps + p.split - 1) / p.split) * BK);
    p.grid = dim3((unsigned)((m.rows + kBN - 1) / kBN), (unsigned)((rows + kBM - 1) / kBM), (unsigned)p.split);
    return p;
}

// The LDS-ring tile (qmm_dma_kernel) takes X whenever a lane's scales of a
// super-step fill whole dwords (group size 32 or 64, or 128 with fp32 scales);
// fp32 X is first rounded to bf16 into the workspace (as the register tile
// rounds it on its way to LDS, so both give the same bits).
bool qmm_dma_ok(const QuantMatrix& m, int x_dtype) {
    (void)x_dtype;
    const int gl = log2_exact(m.group_size);
    return gl == 5 || gl == 6 || (gl == 7 && m.sb_dtype == JH_F32);
}

// Bytes of the bf16 copy of fp32 X in the workspace, rounded up to 256.
size_t qmm_xconv_bytes(int64_t rows, int64_t in) { return ((size_t)rows * (size_t)in * 2 + 255) & ~(size_t)255; }

// n fp32 values (16-byte aligned, n a multiple of 4) to bf16, round to nearest even.
__global__ void x_to_bf16_kernel(const float4* __restrict__ x, int64_t n4, uint2* __restrict__ out) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
        const float4 v = x[i];
        out[i] = make_uint2(pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w));
    }
}

bool qmm_uses_mfma(const QuantMatrix& m, int64_t rows, int x_dtype) {
    const int gl = log2_exact(m.group_size);
    const int64_t xb = x_dtype == JH_F32 ? 4 : 2;
    return m.bits == 4 && gl >= 5 && gl <= 7 && (m.in % BK) == 0 && (m.in % m.group_size) == 0 &&
           (m.rows + 256) * (m.in / 2) < ((int64_t)1 << 31) && (rows + 512) * m.in * xb < ((int64_t)1 << 31);
}

size_t qmm_workspace_bytes(const QuantMatrix& m, int64_t rows, int x_dtype, int y_dtype, int num_cus,
                           bool in_launch) {
    (void)y_dtype;
    if (!qmm_uses_mfma(m, rows, x_dtype)) return 0;
    const QmmPlan p = qmm_plan(m, rows, num_cus, qmm_dma_ok(m, x_dtype), in_launch);
    const size_t xconv = p.wreg && p.lead > 0 && x_dtype == JH_F32 ? qmm_xconv_bytes(rows, m.in) : 0;
    return xconv + (p.split == 1 ? 0 : sizeof(float) * (size_t)p.split * split_stride((uint32_t)rows, (uint32_t)m.rows));
}

template <int NW, int WNF, int SUP, bool SPLIT, bool XF32>
void launch_tile_wreg(const QuantMatrix& m, const void* x, int64_t rows, void* y, int y_dtype, int gl,
                      uint32_t k_per_split, float* acc, dim3 grid, hipStream_t st) {
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, dim3(64 * NW), 0, st, m.w, m.scales, m.biases, x, y, y_dtype,
                           (uint32_t)rows, (uint32_t)m.rows, (uint32_t)m.in, k_per_split, acc);
    };
    auto by_gs = [&](auto sbt) {
        constexpr int SBT = decltype(sbt)::value;
        if (gl == 5) go(qmm_wreg_kernel<SPLIT, XF32, SBT, 5, NW, WNF, SUP>);
        else if (gl == 6) go(qmm_wreg_kernel<SPLIT, XF32, SBT, 6, NW, WNF, SUP>);
        else go(qmm_wreg_kernel<SPLIT, XF32, SBT, 7, NW, WNF, SUP>);
    };
    if (m.sb_dtype == JH_F32)
        by_gs(std::integral_constant<int, 2>{});
    else if (m.sb_dtype == JH_F16)
        by_gs(std::integral_constant<int, 1>{});
    else
        by_gs(std::integral_constant<int, 0>{});
}

template <int NW, int A, bool SPLIT, int RB = RBM, bool INL = false>
void launch_tile_dma(const QuantMatrix& m, const void* x, int64_t rows, void* y, int y_dtype, int gl,
                     uint32_t k_per_split, float* acc, dim3 grid, hipStream_t st, InLaunchSync sy = {}) {
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, dim3(64 * NW), 0, st, m.w, m.scales, m.biases, x, y, y_dtype,
                           (uint32_t)rows, (uint32_t)m.rows, (uint32_t)m.in, k_per_split, acc, sy);
    };
    auto by_gs = [&](auto sbt) {
        constexpr int SBT = decltype(sbt)::value;
        if (gl == 5) go(qmm_dma_kernel<SPLIT, SBT, 5, NW, A, RB, INL>);
        else if (gl == 6) go(qmm_dma_kernel<SPLIT, SBT, 6, NW, A, RB, INL>);
        else if constexpr (SBT == 2) go(qmm_dma_kernel<SPLIT, SBT, 7, NW, A, RB, INL>);
    };
    if (m.sb_dtype == JH_F32)
        by_gs(std::integral_constant<int, 2>{});
    else if (m.sb_dtype == JH_F16)
        by_gs(std::integral_constant<int, 1>{});
    else
        by_gs(std::integral_constant<int, 0>{});
}

template <bool SPLIT, bool XF32>
void launch_tile(const QuantMatrix& m, const void* x, int64_t rows, void* y, int y_dtype, int gl,
                 uint32_t k_per_split, float* acc, dim3 grid, hipStream_t st) {
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, dim3(NT), 0, st, m.w, m.scales, m.biases, x, y, y_dtype,
                           (uint32_t)rows, (uint32_t)m.rows, (uint32_t)m.in, gl, k_per_split, acc);
    };
    if (m.sb_dtype == JH_F32)
        go(qmm_mfma_kernel<SPLIT, XF32, 2>);
    else if (m.sb_dtype == JH_F16)
        go(qmm_mfma_kernel<SPLIT, XF32, 1>);
    else
        go(qmm_mfma_kernel<SPLIT, XF32, 0>);
}

Status launch_qmm(const QuantMatrix& m, const void* x, int x_dtype, int64_t rows, void* y,
                  int y_dtype, int num_cus, hipStream_t st, void* workspace, InLaunchSync sync) {
    if (!qmm_uses_mfma(m, rows, x_dtype)) return launch_generic(m, x, x_dtype, rows, y, y_dtype, num_cus, st);
    const int gl = log2_exact(m.group_size);
    const bool dma = qmm_dma_ok(m, x_dtype);
    const QmmPlan p = qmm_plan(m, rows, num_cus, dma, sync.counters != nullptr);
    const bool xf32 = x_dtype == JH_F32;
    char* ws = static_cast<char*>(workspace);
    if (p.wreg && p.lead > 0 && xf32) {
        // the LDS-ring tile reads bf16 X: round fp32 X into the workspace first
        if (!ws) return Status::fail(JH_ERR_INVALID, "qmm: fp32 x needs a workspace");
        const int64_t n4 = rows * m.in / 4;  // in is a multiple of 256
        hipLaunchKernelGGL(x_to_bf16_kernel, dim3((unsigned)std::min<int64_t>((n4 + 255) / 256, 4096)), dim3(256), 0,
                           st, static_cast<const float4*>(x), n4, reinterpret_cast<uint2*>(ws));
        x = ws;
        ws += qmm_xconv_bytes(rows, m.in);
    }
    auto tile = [&](auto split_c, float* acc) {
        constexpr bool SPLIT = decltype(split_c)::value;
        if (p.wreg && p.lead > 0 && p.rb == 256) {
            launch_tile_dma<8, 1, SPLIT, 256>(m, x, rows, y, y_dtype, gl, p.k_per_split, acc, p.grid, st);
        } else if (p.wreg && p.lead > 0 && p.rb == 32) {
            if (p.nw == 8)
                launch_tile_dma<8, 3, SPLIT, 32>(m, x, rows, y, y_dtype, gl, p.k_per_split, acc, p.grid, st);
            else
                launch_tile_dma<4, 3, SPLIT, 32>(m, x, rows, y, y_dtype, gl, p.k_per_split, acc, p.grid, st);
        } else if (p.wreg && p.lead > 0 && p.rb == 64) {
            if (p.nw == 8)
                launch_tile_dma<8, 2, SPLIT, 64>(m, x, rows, y, y_dtype, gl, p.k_per_split, acc, p.grid, st);
            else
                launch_tile_dma<4, 2, SPLIT, 64>(m, x, rows, y, y_dtype, gl, p.k_per_split, acc, p.grid, st);
        } else if (p.wreg && p.lead > 0) {
            if (p.nw == 8)
                launch_tile_dma<8, 3, SPLIT>(m, x, rows, y, y_dtype, gl, p.k_per_split, acc, p.grid, st);
            else if (p.lead == 3)
                launch_tile_dma<4, 3, SPLIT>(m, x, rows, y, y_dtype, gl, p.k_per_split, acc, p.grid, st);
            else
                launch_tile_dma<4, 1, SPLIT>(m, x, rows, y, y_dtype, gl, p.k_per_split, acc, p.grid, st);
        } else if (p.wreg) {
            if (p.nw == 6) {
                if (xf32) launch_tile_wreg<6, 1, 256, SPLIT, true>(m, x, rows, y, y_dtype, gl, p.k_per_split, acc, p.grid, st);
                else launch_tile_wreg<6, 1, 256, SPLIT, false>(m, x, rows, y, y_dtype, gl, p.k_per_split, acc, p.grid, st);
            } else if (p.nw == 8) {
                if (xf32) launch_tile_wreg<8, 1, 256, SPLIT, true>(m, x, rows, y, y_dtype, gl, p.k_per_split, acc, p.grid, st);
                else launch_tile_wreg<8, 1, 256, SPLIT, false>(m, x, rows, y, y_dtype, gl, p.k_per_split, acc, p.grid, st);
            } else {
                if (xf32) launch_tile_wreg<4, 1, 256, SPLIT, true>(m, x, rows, y, y_dtype, gl, p.k_per_split, acc, p.grid, st);
                else launch_tile_wreg<4, 1, 256, SPLIT, false>(m, x, rows, y, y_dtype, gl, p.k_per_split, acc, p.grid, st);
            }
        } else {
            if (xf32) launch_tile<SPLIT, true>(m, x, rows, y, y_dtype, gl, p.k_per_split, acc, p.grid, st);
            else launch_tile<SPLIT, false>(m, x, rows, y, y_dtype, gl, p.k_per_split, acc, p.grid, st);
        }
    };
    if (p.split == 1) {
        tile(std::false_type{}, nullptr);
        return Status::ok();
    }
    // split K: each K range stores its fp32 partial tile into its own slice of
    // the workspace, and the slices are added in order into y, inside the launch
    // or by a pass of its own
    float* acc = reinterpret_cast<float*>(ws);
    if (!acc) return Status::fail(JH_ERR_INVALID, "qmm: split-K needs a workspace");
    const int64_t n = rows * m.rows;
    if (p.inl && (reinterpret_cast<uintptr_t>(y) & (y_dtype == JH_F32 ? 15 : 7)) == 0) {
        // (qmm_inl_fits holds for the plan; y takes whole 4-column items)
        if (p.lead == 3)
            launch_tile_dma<4, 3, true, 128, true>(m, x, rows, y, y_dtype, gl, p.k_per_split, acc, p.grid, st, sync);
        else
            launch_tile_dma<4, 1, true, 128, true>(m, x, rows, y, y_dtype, gl, p.k_per_split, acc, p.grid, st, sync);
        return Status::ok();
    }
    tile(std::true_type{}, acc);
    hipLaunchKernelGGL(split_sum_kernel, dim3((unsigned)std::min<int64_t>((n / 4 + 255) / 256 + 1, 4096)), dim3(256),
                       0, st, acc, (int)p.split, n, y, y_dtype);
    return Status::ok();
}

}  // namespace jh
