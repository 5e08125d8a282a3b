// Prefill GEMM for MLX affine 4-bit weights on gfx950:
//   Y[M, N] = X[M, K] . W^T,  W dequantized tile by tile into LDS as bf16.
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
// When the tile grid is too small to fill the GPU, K is split over blockIdx.z
// and the partial tiles are added with fp32 atomics into an fp32 buffer.
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
// Even codes (0,2,4,6) sit one per byte of lo, odd codes (1,3,5,7) of hi;
// v_cvt_f32_ubyte0..3 widen them without shifts.
__device__ __forceinline__ void store_w(uint32_t word, float sc, float bi, uint8_t* buf, int tid, int j) {
    uint8_t* ws = buf + BM * ROW_BYTES;
    const uint32_t lo = word & 0x0F0F0F0Fu, hi = (word >> 4) & 0x0F0F0F0Fu;
    uint32_t o[4];
#pragma unroll
    for (int bsel = 0; bsel < 4; bsel++) {
        const float qe = (float)((lo >> (8 * bsel)) & 0xFFu);
        const float qo = (float)((hi >> (8 * bsel)) & 0xFFu);
        o[bsel] = (uint32_t)f32_to_bf16_hw(fmaf(qe, sc, bi)) | ((uint32_t)f32_to_bf16_hw(fmaf(qo, sc, bi)) << 16);
    }
    const int row = tid >> 2, chunk = 2 * (tid & 3) + j;
    *reinterpret_cast<uint4*>(ws + swz(row, chunk)) = make_uint4(o[0], o[1], o[2], o[3]);
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
                        atomicAdd(acc_out + (size_t)m * N + n, acc[i][j][r]);
                    else
                        store_y(Y, (int64_t)m * N + n, acc[i][j][r], y_dt);
                }
            }
        }
}

__global__ void zero_f32_kernel(float* __restrict__ p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = 0.0f;
}

__global__ void f32_to_y_kernel(const float* __restrict__ a, void* __restrict__ y, int y_dt, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        store_y(y, i, a[i], y_dt);
}

int log2_exact(int v) {
    int l = 0;
    while ((1 << l) < v) l++;
    return ((1 << l) == v) ? l : -1;
}

}  // namespace

Status launch_generic(const QuantMatrix& m, const void* x, int x_dtype, int64_t rows, void* y,
                      int y_dtype, int num_cus, hipStream_t st);

constexpr int kBM = BM, kBN = BN;  // tile used by the launcher

int64_t qmm_split(const QuantMatrix& m, int64_t rows, int num_cus) {
    const int64_t tiles = ((m.rows + kBN - 1) / kBN) * ((rows + kBM - 1) / kBM);
    const int64_t ksteps = m.in / BK;
    int64_t split = 1;
    // aim for two tiles per CU, keep at least 8 K steps per split
    while (tiles * split < 2 * num_cus && ksteps / (split * 2) >= 8) split *= 2;
    return split;
}

bool qmm_uses_mfma(const QuantMatrix& m, int64_t rows, int x_dtype) {
    const int gl = log2_exact(m.group_size);
    const int64_t xb = x_dtype == JH_F32 ? 4 : 2;
    return gl >= 5 && gl <= 7 && (m.in % BK) == 0 && (m.in % m.group_size) == 0 &&
           (m.rows + 256) * (m.in / 2) < ((int64_t)1 << 31) && (rows + 512) * m.in * xb < ((int64_t)1 << 31);
}

size_t qmm_workspace_bytes(const QuantMatrix& m, int64_t rows, int x_dtype, int y_dtype, int num_cus) {
    if (!qmm_uses_mfma(m, rows, x_dtype) || qmm_split(m, rows, num_cus) == 1 || y_dtype == JH_F32) return 0;
    return sizeof(float) * (size_t)(rows * m.rows);
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
                  int y_dtype, int num_cus, hipStream_t st, void* workspace) {
    if (!qmm_uses_mfma(m, rows, x_dtype)) return launch_generic(m, x, x_dtype, rows, y, y_dtype, num_cus, st);
    const int gl = log2_exact(m.group_size);
    const int64_t split = qmm_split(m, rows, num_cus);
    const int64_t ksteps = m.in / BK;
    const uint32_t k_per_split = (uint32_t)(((ksteps + split - 1) / split) * BK);
    const dim3 grid((unsigned)((m.rows + kBN - 1) / kBN), (unsigned)((rows + kBM - 1) / kBM), (unsigned)split);
    const bool xf32 = x_dtype == JH_F32;
    if (split == 1) {
        if (xf32)
            launch_tile<false, true>(m, x, rows, y, y_dtype, gl, k_per_split, nullptr, grid, st);
        else
            launch_tile<false, false>(m, x, rows, y, y_dtype, gl, k_per_split, nullptr, grid, st);
        return Status::ok();
    }
    // split K: fp32 partial tiles meet by atomic adds (in y itself when y is fp32)
    float* acc = y_dtype == JH_F32 ? static_cast<float*>(y) : static_cast<float*>(workspace);
    if (!acc) return Status::fail(JH_ERR_INVALID, "qmm: split-K needs a workspace");
    const int64_t n = rows * m.rows;
    hipLaunchKernelGGL(zero_f32_kernel, dim3((unsigned)std::min<int64_t>((n + 255) / 256, 8192)), dim3(256),
                       0, st, acc, n);
    if (xf32)
        launch_tile<true, true>(m, x, rows, y, y_dtype, gl, k_per_split, acc, grid, st);
    else
        launch_tile<true, false>(m, x, rows, y, y_dtype, gl, k_per_split, acc, grid, st);
    if (y_dtype != JH_F32)
        hipLaunchKernelGGL(f32_to_y_kernel, dim3((unsigned)std::min<int64_t>((n + 255) / 256, 8192)),
                           dim3(256), 0, st, acc, y, y_dtype, n);
    return Status::ok();
}

}  // namespace jh
