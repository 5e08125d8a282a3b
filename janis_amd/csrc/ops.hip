// The engine operators around the quantized products that the model code
// calls as they are (qwen/moe.go:455-510 before any fusion): Softmax, Mean,
// ScalarMul/ScalarAdd, QuantMatmul/GatherQuantMatmul with transpose = false,
// and the NaN/Inf read-back count of the value checks.
//
// None of these is on the decode hot path of the target models; they keep the
// CPU backend's arithmetic order so results match it bit for bit where its
// order is sequential.
#include "jh_common.hpp"

namespace jh {
namespace {

__device__ __forceinline__ float load_act(const void* p, int64_t i, int dt) {
    return dt == JH_BF16 ? bf16_to_f32(static_cast<const uint16_t*>(p)[i]) : static_cast<const float*>(p)[i];
}

// ---- QuantMatmul / GatherQuantMatmul with transpose = false ----------------------
// The CPU backend computes MatMul(x, Dequantize(w)) (cpu/cpu_misc.go:233-236):
// y[r, j] = sum_n x[r, n] * W[n, j] over the n = out_features rows of W, in
// increasing n, skipping x[r, n] == 0, each term rounded and then added
// (cpu/cpu_ops.go:39-48), with W[n, j] = fl32(q * s) + b (cpu/cpu_misc.go:154-156).
// One thread owns one packed word (32/bits consecutive columns) of one output
// row and walks n in that order, so each output has the CPU backend's bits.
// Gather mode (idx != nullptr): output row r is slot r of the (lead, slot)
// pairs, its x row is lead * A + (A == 1 ? 0 : slot) and its W the stack's
// expert idx[r] (an index outside [0, n_experts) gives a row of NaN).
template <int BITS>
__global__ __launch_bounds__(256) void qmt_kernel(const uint32_t* __restrict__ W, const void* __restrict__ S,
                                                  const void* __restrict__ B, int sb_dt, const void* __restrict__ X,
                                                  int x_dt, void* __restrict__ Y, int y_dt, int64_t N, int64_t K,
                                                  int gs, int64_t rows, const int32_t* __restrict__ idx,
                                                  int64_t n_experts, int64_t k_slots, int64_t a_vectors) {
#pragma clang fp contract(off)
    constexpr int VPW = 32 / BITS;
    constexpr uint32_t MASK = (1u << BITS) - 1u;
    const int64_t P = K / VPW, G = K / gs;
    const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (p >= P) return;
    for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
        int64_t xrow = r, e = 0;
        if (idx) {
            const int64_t l = r / k_slots, k = r % k_slots;
            xrow = l * a_vectors + (a_vectors == 1 ? 0 : k);
            e = idx[r];
            if (e < 0 || e >= n_experts) {
                for (int l2 = 0; l2 < VPW; l2++) store_y(Y, r * K + p * VPW + l2, __builtin_nanf(""), y_dt);
                continue;
            }
        }
        const uint32_t* We = W + e * N * P;
        const int64_t sb0 = e * N * G;
        float acc[VPW];
#pragma unroll
        for (int l = 0; l < VPW; l++) acc[l] = 0.0f;
        for (int64_t n = 0; n < N; n++) {
            const float a = load_act(X, xrow * N + n, x_dt);
            if (a == 0.0f) continue;
            const uint32_t word = We[n * P + p];
#pragma unroll
            for (int l = 0; l < VPW; l++) {
                const int64_t g = (p * VPW + l) / gs;
                const float s = load_sb(S, sb0 + n * G + g, sb_dt);
                const float b = load_sb(B, sb0 + n * G + g, sb_dt);
                const float w = (float)((word >> (BITS * l)) & MASK) * s + b;
                acc[l] = acc[l] + a * w;
            }
        }
#pragma unroll
        for (int l = 0; l < VPW; l++) store_y(Y, r * K + p * VPW + l, acc[l], y_dt);
    }
}

// ---- Softmax (cpu/cpu.go:461-499) ------------------------------------------------
// One block per line along the axis of an [outer, len, inner] view: the maximum,
// e_i = fl32(exp(double(x_i - max))), their sum, then e_i / sum. The sum is the
// CPU backend's sequential fp32 sum (one lane, in order, from LDS) for lines of
// up to kSoftmaxSeq; longer lines (beyond any router width) sum in a tree.
constexpr int kSoftmaxSeq = 8192;

__global__ __launch_bounds__(256) void softmax_kernel(const void* __restrict__ X, int x_dt, float* __restrict__ Y,
                                                      int64_t lines, int64_t len, int64_t inner) {
    __shared__ float e_lds[kSoftmaxSeq];
    __shared__ float red[4];
    __shared__ float tot;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    for (int64_t line = blockIdx.x; line < lines; line += gridDim.x) {
        const int64_t base = (line / inner) * len * inner + line % inner;
        float mx = -__builtin_inff();
        for (int64_t i = threadIdx.x; i < len; i += 256) mx = fmaxf(mx, load_act(X, base + i * inner, x_dt));
        mx = wave_max(mx);
        if (lane == 0) red[wv] = mx;
        __syncthreads();
        mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        __syncthreads();
        float part = 0.0f;
        for (int64_t i = threadIdx.x; i < len; i += 256) {
            const float e = (float)exp((double)(load_act(X, base + i * inner, x_dt) - mx));
            if (len <= kSoftmaxSeq) e_lds[i] = e;
            else Y[base + i * inner] = e;
            part += e;
        }
        if (len <= kSoftmaxSeq) {
            __syncthreads();
            if (threadIdx.x == 0) {
                float s = 0.0f;
                for (int64_t i = 0; i < len; i++) s += e_lds[i];
                tot = s;
            }
            __syncthreads();
            const float sum = tot;
            for (int64_t i = threadIdx.x; i < len; i += 256) Y[base + i * inner] = e_lds[i] / sum;
        } else {
            part = wave_sum(part);
            if (lane == 0) red[wv] = part;
            __syncthreads();
            const float sum = (red[0] + red[1]) + (red[2] + red[3]);
            // each thread rescales the exponentials it wrote itself
            for (int64_t i = threadIdx.x; i < len; i += 256) Y[base + i * inner] = Y[base + i * inner] / sum;
        }
        __syncthreads();
    }
}

// ---- Mean over an axis (cpu/cpu_ops.go:113-142) ------------------------------------
// One thread per output: the sequential fp32 sum along the axis, then / len.
__global__ __launch_bounds__(256) void mean_kernel(const void* __restrict__ X, int x_dt, float* __restrict__ Y,
                                                   int64_t outs, int64_t len, int64_t inner) {
    for (int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x; o < outs; o += (int64_t)gridDim.x * 256) {
        const int64_t base = (o / inner) * len * inner + o % inner;
        float s = 0.0f;
        for (int64_t i = 0; i < len; i++) s += load_act(X, base + i * inner, x_dt);
        Y[o] = s / (float)len;
    }
}

// ---- ScalarMul / ScalarAdd (cpu/cpu_misc.go:24-30) ----------------------------------
__global__ __launch_bounds__(256) void scalar_kernel(int op, const void* __restrict__ X, int x_dt, float v,
                                                     void* __restrict__ Y, int y_dt, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const float a = load_act(X, i, x_dt);
        store_y(Y, i, op == JH_SCALAR_MUL ? a * v : a + v, y_dt);
    }
}

// ---- NaN/Inf count (the read-back check of ggml/ggml.go:622-677) -----------------
// res[0] += count of non-finite values, res[1] = min index of one (n when none).
__global__ __launch_bounds__(256) void nonfinite_kernel(const void* __restrict__ X, int x_dt, int64_t n,
                                                        unsigned long long* __restrict__ res) {
    unsigned long long cnt = 0, first = (unsigned long long)n;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const uint32_t u = x_dt == JH_BF16 ? (uint32_t)static_cast<const uint16_t*>(X)[i] << 16
                         : x_dt == JH_F16  ? __float_as_uint(f16_to_f32(static_cast<const uint16_t*>(X)[i]))
                                           : static_cast<const uint32_t*>(X)[i];
        if ((u & 0x7f800000u) == 0x7f800000u) {
            cnt++;
            if ((unsigned long long)i < first) first = (unsigned long long)i;
        }
    }
    if (cnt) {
        atomicAdd(&res[0], cnt);
        atomicMin(&res[1], first);
    }
}

int64_t grid_for(int64_t n, int64_t cap) { return std::max<int64_t>(1, std::min<int64_t>((n + 255) / 256, cap)); }

}  // namespace

Status launch_quant_matmul_t(const QuantMatrix& m, const void* x, int x_dtype, int64_t rows, void* y, int y_dtype,
                             const int32_t* idx, int64_t n_experts, int64_t k_slots, int64_t a_vectors,
                             hipStream_t st) {
    const int64_t P = m.in * m.bits / 32;
    const dim3 grid((unsigned)((P + 255) / 256), (unsigned)std::min<int64_t>(rows, 65535));
#define JH_QMT(BITS)                                                                                            \
    hipLaunchKernelGGL(qmt_kernel<BITS>, grid, dim3(256), 0, st, m.w, m.scales, m.biases, m.sb_dtype, x, x_dtype, \
                       y, y_dtype, m.rows, m.in, m.group_size, rows, idx, n_experts, k_slots, a_vectors)
    if (m.bits == 2) JH_QMT(2);
    else if (m.bits == 4) JH_QMT(4);
    else if (m.bits == 8) JH_QMT(8);
    else return Status::fail(JH_ERR_UNSUPPORTED, "quant_matmul_t: bits must be 2, 4 or 8");
#undef JH_QMT
    return Status::ok();
}

Status launch_softmax(const void* x, int x_dt, float* y, int64_t outer, int64_t len, int64_t inner, hipStream_t st) {
    const int64_t lines = outer * inner;
    if (lines == 0 || len == 0) return Status::ok();
    hipLaunchKernelGGL(softmax_kernel, dim3((unsigned)std::min<int64_t>(lines, 1 << 20)), dim3(256), 0, st, x, x_dt,
                       y, lines, len, inner);
    return Status::ok();
}

Status launch_mean(const void* x, int x_dt, float* y, int64_t outer, int64_t len, int64_t inner, hipStream_t st) {
    const int64_t outs = outer * inner;
    if (outs == 0) return Status::ok();
    hipLaunchKernelGGL(mean_kernel, dim3((unsigned)grid_for(outs, 1 << 16)), dim3(256), 0, st, x, x_dt, y, outs, len,
                       inner);
    return Status::ok();
}

Status launch_scalar(int op, const void* x, int x_dt, float v, void* y, int y_dt, int64_t n, hipStream_t st) {
    if (n == 0) return Status::ok();
    hipLaunchKernelGGL(scalar_kernel, dim3((unsigned)grid_for(n, 1 << 16)), dim3(256), 0, st, op, x, x_dt, v, y, y_dt,
                       n);
    return Status::ok();
}

Status launch_nonfinite(const void* x, int x_dt, int64_t n, unsigned long long* res, hipStream_t st) {
    if (n == 0) return Status::ok();
    hipLaunchKernelGGL(nonfinite_kernel, dim3((unsigned)grid_for(n, 4096)), dim3(256), 0, st, x, x_dt, n, res);
    return Status::ok();
}

}  // namespace jh
