// Prefill GEMM for MLX affine 4-bit weights on gfx950:
//   Y[M, N] = X[M, K] . W^T,  W dequantized tile by tile into LDS as bf16.
//
// Reference semantics: QuantMatmul with rows > 1 (cpu/cpu_misc.go:378-399),
// which dequantizes a weight row once (wbuf = q*scale + bias) and dots it with
// every x row in fp32. Here each 64-wide K step (one quantization group for
// group size 64) stages
//   * an X tile [BM x 64] as bf16 (converted on the fly if X is fp32), and
//   * a W tile [BN x 64]: 128-bit loads of packed words, dequantized in
//     registers as fma(q, scale, bias) (exactly fl32(q*scale+bias) for bf16
//     scales) and rounded to bf16,
// into LDS, then four waves each compute a 64x64 block of Y with
// v_mfma_f32_32x32x16_bf16 (fp32 accumulation). LDS rows are padded by 16 bytes
// so the 16-byte fragment reads of 16 consecutive rows hit distinct banks.
// Operand layout of the 32x32x16 MFMA used below: lane l supplies
//   A[i = l % 32][k = 8*(l/32) .. +8]  and  B[k = 8*(l/32) .. +8][j = l % 32],
// and accumulator register r of lane l holds D[8*(r/4) + 4*(l/32) + r%4][l % 32].
#include "jh_common.hpp"

namespace jh {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int BK = 64;
constexpr int LDK = BK + 8;  // padded LDS row, in bf16 elements (144 bytes)

template <int BM, int BN>
__global__ __launch_bounds__(256) void qmm_mfma_kernel(
    const uint32_t* __restrict__ W, const void* __restrict__ S, const void* __restrict__ B,
    int sb_dt, const void* __restrict__ X, int x_dt, void* __restrict__ Y, int y_dt, int64_t M,
    int64_t N, int64_t K, int gs_log2) {
    static_assert(BM == 128 && BN == 128, "tile loader assumes 128x128 with 256 threads");
    __shared__ __attribute__((aligned(16))) uint16_t As[BM * LDK];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[BN * LDK];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
    const int wm = wave >> 1, wn = wave & 1;
    const int64_t P = K >> 3, G = K >> gs_log2;

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    const int ld_row = tid >> 1, ld_half = tid & 1;

    for (int64_t k0 = 0; k0 < K; k0 += BK) {
        // ---- X tile: thread -> (row, 32-element half) --------------------------
        {
            const int64_t m = m0 + ld_row;
            uint4 v[4];
            if (m < M) {
                if (x_dt == JH_BF16) {
                    const uint4* src = reinterpret_cast<const uint4*>(
                        static_cast<const uint16_t*>(X) + m * K + k0 + 32 * ld_half);
#pragma unroll
                    for (int j = 0; j < 4; j++) v[j] = src[j];
                } else {
                    const float4* src = reinterpret_cast<const float4*>(
                        static_cast<const float*>(X) + m * K + k0 + 32 * ld_half);
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const float4 a = src[2 * j], b = src[2 * j + 1];
                        v[j] = make_uint4(pack_bf16x2(a.x, a.y), pack_bf16x2(a.z, a.w),
                                          pack_bf16x2(b.x, b.y), pack_bf16x2(b.z, b.w));
                    }
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++) v[j] = make_uint4(0, 0, 0, 0);
            }
            uint4* dst = reinterpret_cast<uint4*>(As + ld_row * LDK + 32 * ld_half);
#pragma unroll
            for (int j = 0; j < 4; j++) dst[j] = v[j];
        }
        // ---- W tile: 4 words (32 codes, one group for gs >= 32) per thread -------
        {
            const int64_t n = n0 + ld_row;
            uint4 wq = make_uint4(0, 0, 0, 0);
            float s = 0.0f, b = 0.0f;
            if (n < N) {
                wq = *reinterpret_cast<const uint4*>(W + n * P + (k0 >> 3) + 4 * ld_half);
                const int64_t g = (k0 + 32 * ld_half) >> gs_log2;
                s = load_sb(S, n * G + g, sb_dt);
                b = load_sb(B, n * G + g, sb_dt);
            }
            const uint32_t words[4] = {wq.x, wq.y, wq.z, wq.w};
            uint4* dst = reinterpret_cast<uint4*>(Bs + ld_row * LDK + 32 * ld_half);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t w = words[j];
                uint32_t o[4];
#pragma unroll
                for (int l = 0; l < 8; l += 2) {
                    const float a0 = fmaf((float)((w >> (4 * l)) & 0xFu), s, b);
                    const float a1 = fmaf((float)((w >> (4 * l + 4)) & 0xFu), s, b);
                    o[l / 2] = pack_bf16x2(a0, a1);
                }
                dst[j] = make_uint4(o[0], o[1], o[2], o[3]);
            }
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < BK / 16; kk++) {
            bf16x8_t a[2], bb[2];
            const int kof = kk * 16 + 8 * (lane >> 5);
#pragma unroll
            for (int i = 0; i < 2; i++)
                a[i] = *reinterpret_cast<const bf16x8_t*>(As + (wm * 64 + 32 * i + (lane & 31)) * LDK + kof);
#pragma unroll
            for (int j = 0; j < 2; j++)
                bb[j] = *reinterpret_cast<const bf16x8_t*>(Bs + (wn * 64 + 32 * j + (lane & 31)) * LDK + kof);
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], bb[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int64_t n = n0 + wn * 64 + 32 * j + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int64_t m = m0 + wm * 64 + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < M && n < N) store_y(Y, m * N + n, acc[i][j][r], y_dt);
            }
        }
}

int log2_exact(int v) {
    int l = 0;
    while ((1 << l) < v) l++;
    return ((1 << l) == v) ? l : -1;
}

}  // namespace

Status launch_generic(const QuantMatrix& m, const void* x, int x_dtype, int64_t rows, void* y,
                      int y_dtype, int num_cus, hipStream_t st);

Status launch_qmm(const QuantMatrix& m, const void* x, int x_dtype, int64_t rows, void* y,
                  int y_dtype, int num_cus, hipStream_t st) {
    const int gl = log2_exact(m.group_size);
    const bool mfma_ok = gl >= 5 && gl <= 7 && (m.in % BK) == 0 && (m.in % m.group_size) == 0;
    if (!mfma_ok) return launch_generic(m, x, x_dtype, rows, y, y_dtype, num_cus, st);
    const dim3 grid((unsigned)((m.rows + 127) / 128), (unsigned)((rows + 127) / 128));
    hipLaunchKernelGGL((qmm_mfma_kernel<128, 128>), grid, dim3(256), 0, st, m.w, m.scales,
                       m.biases, m.sb_dtype, x, x_dtype, y, y_dtype, rows, m.rows, m.in, gl);
    return Status::ok();
}

}  // namespace jh
