// Dequantize (cpu/cpu_misc.go:134-161): out[r, j] = fl32(q(r,j) * scale + bias).
//
// One thread per packed word; its 32/bits codes are written with 8- or 16-byte
// stores. The product q*scale is rounded before the bias
// is added, the reference's order, so the result is bit-identical for any
// scale dtype (for bf16 and f16 scales q*scale is exact and a fused
// multiply-add would agree as well; for fp32 scales it would not).
// Memory-bound: reads 4 B + scale/bias per word, writes 4 B per output (fp32).
#include "jh_common.hpp"

namespace jh {
namespace {

// One thread per packed word of BITS-wide codes (VPW = 32/BITS per word).
template <int BITS>
__global__ __launch_bounds__(256) void dequant_kernel(const uint32_t* __restrict__ W,
                                                      const void* __restrict__ S,
                                                      const void* __restrict__ B, int sb_dt,
                                                      void* __restrict__ out, int out_dt,
                                                      int64_t rows, int64_t P, int gs) {
    constexpr int VPW = 32 / BITS;
    constexpr uint32_t MASK = (1u << BITS) - 1u;
    const int64_t total = rows * P;
    const int64_t K = P * VPW, G = K / gs;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        const int64_t r = i / P, p = i - r * P;
        const uint32_t word = W[i];
        float v[VPW];
        const int64_t g0 = (VPW * p) / gs;
        float s = load_sb(S, r * G + g0, sb_dt), b = load_sb(B, r * G + g0, sb_dt);
        int64_t gcur = g0;
#pragma unroll
        for (int l = 0; l < VPW; l++) {
            const int64_t g = (VPW * p + l) / gs;
            if (g != gcur) {  // only for groups smaller than a word
                gcur = g;
                s = load_sb(S, r * G + g, sb_dt);
                b = load_sb(B, r * G + g, sb_dt);
            }
            v[l] = unfused_qsb((float)((word >> (BITS * l)) & MASK), s, b);
        }
        if (out_dt == JH_BF16) {
            uint32_t o[VPW / 2];
#pragma unroll
            for (int l = 0; l < VPW / 2; l++) o[l] = pack_bf16x2(v[2 * l], v[2 * l + 1]);
            if constexpr (VPW == 4) {
                reinterpret_cast<uint2*>(out)[i] = make_uint2(o[0], o[1]);
            } else {
#pragma unroll
                for (int l = 0; l < VPW / 8; l++)
                    reinterpret_cast<uint4*>(out)[(VPW / 8) * i + l] = make_uint4(o[4 * l], o[4 * l + 1], o[4 * l + 2], o[4 * l + 3]);
            }
        } else {
            float4* o = reinterpret_cast<float4*>(out) + (VPW / 4) * i;
#pragma unroll
            for (int l = 0; l < VPW / 4; l++) o[l] = make_float4(v[4 * l], v[4 * l + 1], v[4 * l + 2], v[4 * l + 3]);
        }
    }
}

}  // namespace

Status launch_dequantize(const QuantMatrix& m, void* out, int out_dtype, hipStream_t st) {
    const int64_t P = m.in * m.bits / 32;
    const int64_t total = m.rows * P;
    if (total == 0) return Status::ok();
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), 0, st, m.w, m.scales, m.biases, m.sb_dtype, out,
                           out_dtype, m.rows, P, m.group_size);
    };
    if (m.bits == 8) go(dequant_kernel<8>);
    else if (m.bits == 2) go(dequant_kernel<2>);
    else go(dequant_kernel<4>);
    return Status::ok();
}

}  // namespace jh
