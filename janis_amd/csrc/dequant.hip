// Dequantize (cpu/cpu_misc.go:134-161): out[r, j] = fl32(q(r,j) * scale + bias).
//
// One thread per packed word; the 8 codes of a word are written as two 16-byte
// stores (fp32) or one (bf16). The product q*scale is rounded before the bias
// is added, the reference's order, so the result is bit-identical for any
// scale dtype (for bf16 and f16 scales q*scale is exact and a fused
// multiply-add would agree as well; for fp32 scales it would not).
// Memory-bound: reads 4 B + scale/bias per 8 outputs, writes 32 B (fp32).
#include "jh_common.hpp"

namespace jh {
namespace {

// fl32(fl32(q * s) + b): the product is rounded before the add, as the
// reference computes it on amd64; contraction into an FMA is switched off here
// (hipcc contracts by default).
__device__ __forceinline__ float unfused_qsb(float q, float s, float b) {
#pragma clang fp contract(off)
    const float p = q * s;
    return p + b;
}

__global__ __launch_bounds__(256) void dequant4_kernel(const uint32_t* __restrict__ W,
                                                       const void* __restrict__ S,
                                                       const void* __restrict__ B, int sb_dt,
                                                       void* __restrict__ out, int out_dt,
                                                       int64_t rows, int64_t P, int gs) {
    const int64_t total = rows * P;
    const int64_t K = P * 8, G = K / gs;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        const int64_t r = i / P, p = i - r * P;
        const uint32_t word = W[i];
        float v[8];
        const int64_t g0 = (8 * p) / gs;
        float s = load_sb(S, r * G + g0, sb_dt), b = load_sb(B, r * G + g0, sb_dt);
        int64_t gcur = g0;
#pragma unroll
        for (int l = 0; l < 8; l++) {
            const int64_t g = (8 * p + l) / gs;
            if (g != gcur) {  // only for group sizes below 8
                gcur = g;
                s = load_sb(S, r * G + g, sb_dt);
                b = load_sb(B, r * G + g, sb_dt);
            }
            v[l] = unfused_qsb((float)((word >> (4 * l)) & 0xFu), s, b);
        }
        if (out_dt == JH_BF16) {
            uint4 o = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                 pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
            reinterpret_cast<uint4*>(out)[i] = o;
        } else {
            float4* o = reinterpret_cast<float4*>(out) + 2 * i;
            o[0] = make_float4(v[0], v[1], v[2], v[3]);
            o[1] = make_float4(v[4], v[5], v[6], v[7]);
        }
    }
}

}  // namespace

Status launch_dequantize(const QuantMatrix& m, void* out, int out_dtype, hipStream_t st) {
    const int64_t P = m.in / 8;
    const int64_t total = m.rows * P;
    if (total == 0) return Status::ok();
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(dequant4_kernel, dim3((unsigned)blocks), dim3(256), 0, st, m.w, m.scales,
                       m.biases, m.sb_dtype, out, out_dtype, m.rows, P, m.group_size);
    return Status::ok();
}

}  // namespace jh
