// The engine.Backend operators of a decode step besides the quantized products,
// on gfx950: RMSNorm (cpu/cpu_ops.go:144-162), RoPE / RoPEFreqs
// (cpu/cpu_attn.go:13-62), SDPA (cpu/cpu_attn.go:64-119), SiLU, Mul, Add
// (cpu/cpu.go:300-329), Argmax (cpu/cpu_misc.go:91-121), row gather (TakeAxis on
// axis 0, cpu/cpu_misc.go:48-89) and the KV-cache append (KVAppender,
// engine/backend.go:56-61).
//
// Activations may be bf16 or fp32 (f16 for the norm weights too); arithmetic is
// fp32, with exp, sqrt, cos, sin and pow evaluated in double where the CPU
// backend does, so results differ from it only by reduction order.
//
// SDPA with one query row per head (decode) is split over the key sequence
// (flash-decoding): block (b*Hk + hk, split) scores its key range for all
// Hq/Hk query heads of kv head hk with an online softmax and writes (max, sum,
// weighted values); a second launch merges the splits. Other shapes take a
// per-query-row kernel with the offset causal mask.
#include "jh_common.hpp"

namespace jh {
namespace {

__device__ __forceinline__ float ld_act(const void* p, int64_t i, int dt) {
    if (dt == JH_BF16) return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
    if (dt == JH_F16) return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
    return static_cast<const float*>(p)[i];
}

__device__ __forceinline__ void st_act(void* p, int64_t i, float v, int dt) {
    if (dt == JH_BF16)
        static_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
    else
        static_cast<float*>(p)[i] = v;
}

// Sum over a block of 256 threads; every thread gets the total.
__device__ float block_sum256(float v, float* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    __syncthreads();
    if (l == 0) red[w] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// ---- RMSNorm: one block per row --------------------------------------------------
__global__ __launch_bounds__(256) void rms_norm_kernel(const void* __restrict__ x, int x_dt,
                                                       const void* __restrict__ w, int w_dt, float eps,
                                                       void* __restrict__ out, int out_dt, int64_t d) {
    __shared__ float red[4];
    const int64_t r = blockIdx.x;
    float ss = 0.0f;
    for (int64_t i = threadIdx.x; i < d; i += 256) {
        const float v = ld_act(x, r * d + i, x_dt);
        ss = fmaf(v, v, ss);
    }
    ss = block_sum256(ss, red);
    const float inv = 1.0f / (float)sqrt((double)(ss / (float)d + eps));
    for (int64_t i = threadIdx.x; i < d; i += 256) {
        const float t = ld_act(x, r * d + i, x_dt) * inv;
        st_act(out, r * d + i, t * ld_act(w, i, w_dt), out_dt);
    }
}

// ---- RoPE: one thread per rotated pair --------------------------------------------
__global__ __launch_bounds__(256) void rope_kernel(const void* __restrict__ x, int x_dt, void* __restrict__ out,
                                                   int out_dt, int64_t rows, int64_t L, int64_t D, int dims,
                                                   int traditional, float base, float scale, int64_t offset,
                                                   const float* __restrict__ freqs) {
    const int half = dims / 2;
    const int64_t per_row = D - half;  // pairs plus pass-through features
    const int64_t total = rows * per_row;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = t / per_row;
        const int i = (int)(t - r * per_row);
        const int64_t o = r * D;
        if (i >= half) {  // features past `dims` pass through
            const int64_t f = dims + (i - half);
            if (f < D) st_act(out, o + f, ld_act(x, o + f, x_dt), out_dt);
            continue;
        }
        const float inv = freqs ? 1.0f / freqs[i] : (float)pow((double)base, -(double)(2 * i) / (double)dims);
        const float pos = (float)(offset + r % L);
        const float theta = pos * scale * inv;
        const float c = (float)cos((double)theta), s = (float)sin((double)theta);
        const int64_t i0 = traditional ? o + 2 * i : o + i;
        const int64_t i1 = traditional ? o + 2 * i + 1 : o + i + half;
        const float a = ld_act(x, i0, x_dt), b = ld_act(x, i1, x_dt);
        st_act(out, i0, a * c - b * s, out_dt);
        st_act(out, i1, a * s + b * c, out_dt);
    }
}

// ---- SDPA, general: one block per (b, h, query row) --------------------------------
// q [B, Hq, Lq, Dh]; k/v [B, Hk, kcap, Dh] with the first Lk rows valid.
__global__ __launch_bounds__(256) void sdpa_rows_kernel(const void* __restrict__ q, int q_dt,
                                                        const void* __restrict__ k, const void* __restrict__ v,
                                                        int kv_dt, void* __restrict__ out, int out_dt, int Hq,
                                                        int Hk, int Lq, int Lk, int kcap, int Dh, float scale,
                                                        int causal) {
    __shared__ float qs[256];
    __shared__ float red[4];
    const int64_t row = blockIdx.x;  // (b*Hq + h)*Lq + i
    const int i = (int)(row % Lq);
    const int64_t bh = row / Lq;
    const int h = (int)(bh % Hq);
    const int64_t b = bh / Hq;
    const int hk = h / (Hq / Hk);
    const int limit = causal ? (Lk - Lq) + i + 1 : Lk;
    const int64_t kbase = (b * Hk + hk) * (int64_t)kcap * Dh;
    for (int d = threadIdx.x; d < Dh; d += 256) qs[d] = ld_act(q, row * Dh + d, q_dt);
    __syncthreads();
    // pass 1: max score (each thread its keys)
    float mx = -__builtin_inff();
    for (int j = threadIdx.x; j < limit; j += 256) {
        float s = 0.0f;
        for (int d = 0; d < Dh; d++) s = fmaf(qs[d], ld_act(k, kbase + (int64_t)j * Dh + d, kv_dt), s);
        mx = fmaxf(mx, s * scale);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    // pass 2: sum of exp and the weighted values, key by key across the block
    float lsum = 0.0f;
    float acc = 0.0f;  // thread d accumulates output feature d (Dh <= 256)
    __shared__ float pj[256];
    for (int j0 = 0; j0 < limit; j0 += 256) {
        const int j = j0 + threadIdx.x;
        float e = 0.0f;
        if (j < limit) {
            float s = 0.0f;
            for (int d = 0; d < Dh; d++) s = fmaf(qs[d], ld_act(k, kbase + (int64_t)j * Dh + d, kv_dt), s);
            e = (float)exp((double)(s * scale - mx));
        }
        lsum += e;
        __syncthreads();
        pj[threadIdx.x] = e;
        __syncthreads();
        const int n = min(256, limit - j0);
        if (threadIdx.x < Dh)
            for (int jj = 0; jj < n; jj++)
                acc = fmaf(pj[jj], ld_act(v, kbase + (int64_t)(j0 + jj) * Dh + threadIdx.x, kv_dt), acc);
    }
    const float sum = block_sum256(lsum, red);
    if (threadIdx.x < Dh) st_act(out, row * Dh + threadIdx.x, acc / sum, out_dt);
}

// ---- SDPA, one query row (decode): split over keys, then merge -------------------
// A wave scores 4 keys per step: 16 lanes per key, 8 features per lane (16-byte
// loads of bf16 keys), partial dots reduced across the 16 lanes with xor
// shuffles so every lane of the group holds the score. Each lane keeps, for every
// query head of the group, a running max, sum and 8 output features.
constexpr int kDecodeMaxGroup = 8;  // query heads per kv head
constexpr int kDecodeDh = 128;

template <int G>
__global__ __launch_bounds__(256) void sdpa_decode_split_kernel(const void* __restrict__ q, int q_dt,
                                                                const uint16_t* __restrict__ k,
                                                                const uint16_t* __restrict__ v, int Hk,
                                                                int Lk, int kcap, float scale, int keys_per_split,
                                                                float* __restrict__ part) {
    constexpr int Dh = kDecodeDh;
    const int bhk = blockIdx.x;  // b*Hk + hk
    const int split = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int kg = lane >> 4, kl = lane & 15;  // key slot in the wave, feature chunk
    const int64_t b = bhk / Hk;
    const int hk = bhk - (int)b * Hk;
    const int Hq = Hk * G;
    float qv[G][8];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < 8; e++)
            qv[g][e] = ld_act(q, ((b * Hq + hk * G + g) * Dh) + 8 * kl + e, q_dt) * scale;
    float m[G], l[G], acc[G][8];
#pragma unroll
    for (int g = 0; g < G; g++) {
        m[g] = -__builtin_inff();
        l[g] = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) acc[g][e] = 0.0f;
    }
    const int j_begin = split * keys_per_split;
    const int j_end = min(Lk, j_begin + keys_per_split);
    const int64_t kbase = (int64_t)bhk * kcap * Dh;
    for (int j = j_begin + wave * 4 + kg; j < j_end; j += 16) {
        const uint4 kr = *reinterpret_cast<const uint4*>(k + kbase + (int64_t)j * Dh + 8 * kl);
        const uint4 vr = *reinterpret_cast<const uint4*>(v + kbase + (int64_t)j * Dh + 8 * kl);
        const float kf[8] = {__uint_as_float(kr.x << 16), __uint_as_float(kr.x & 0xFFFF0000u),
                             __uint_as_float(kr.y << 16), __uint_as_float(kr.y & 0xFFFF0000u),
                             __uint_as_float(kr.z << 16), __uint_as_float(kr.z & 0xFFFF0000u),
                             __uint_as_float(kr.w << 16), __uint_as_float(kr.w & 0xFFFF0000u)};
        const float vf[8] = {__uint_as_float(vr.x << 16), __uint_as_float(vr.x & 0xFFFF0000u),
                             __uint_as_float(vr.y << 16), __uint_as_float(vr.y & 0xFFFF0000u),
                             __uint_as_float(vr.z << 16), __uint_as_float(vr.z & 0xFFFF0000u),
                             __uint_as_float(vr.w << 16), __uint_as_float(vr.w & 0xFFFF0000u)};
#pragma unroll
        for (int g = 0; g < G; g++) {
            float s = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; e++) s = fmaf(qv[g][e], kf[e], s);
#pragma unroll
            for (int o = 8; o > 0; o >>= 1) s += __shfl_xor(s, o, 16);
            const float mn = fmaxf(m[g], s);
            const float corr = __expf(m[g] - mn);
            const float p = __expf(s - mn);
            l[g] = fmaf(l[g], corr, p);
#pragma unroll
            for (int e = 0; e < 8; e++) acc[g][e] = fmaf(acc[g][e], corr, p * vf[e]);
            m[g] = mn;
        }
    }
    // merge the 16 key slots of the block (4 per wave x 4 waves) through LDS
    __shared__ float sm[16][G], sl[16][G], sacc[16][G][Dh];
    const int slot = wave * 4 + kg;
#pragma unroll
    for (int g = 0; g < G; g++) {
        if (kl == 0) {
            sm[slot][g] = m[g];
            sl[slot][g] = l[g];
        }
#pragma unroll
        for (int e = 0; e < 8; e++) sacc[slot][g][8 * kl + e] = acc[g][e];
    }
    __syncthreads();
    // thread t: query head g = t / Dh... (G*Dh <= 1024; 256 threads loop)
    float* dst = part + ((int64_t)bhk * gridDim.y + split) * G * (Dh + 2);
    for (int t = threadIdx.x; t < G * Dh; t += 256) {
        const int g = t / Dh, d = t - g * Dh;
        float M = -__builtin_inff();
        for (int s = 0; s < 16; s++) M = fmaxf(M, sm[s][g]);
        float L = 0.0f, A = 0.0f;
        if (M != -__builtin_inff())
            for (int s = 0; s < 16; s++) {
                const float c = __expf(sm[s][g] - M);
                L = fmaf(sl[s][g], c, L);
                A = fmaf(sacc[s][g][d], c, A);
            }
        dst[g * (Dh + 2) + 2 + d] = A;
        if (d == 0) {
            dst[g * (Dh + 2)] = M;
            dst[g * (Dh + 2) + 1] = L;
        }
    }
}

// Merge the splits of one (b, query head): thread d owns feature d.
__global__ __launch_bounds__(128) void sdpa_decode_merge_kernel(const float* __restrict__ part, int Hk, int G,
                                                                int nsplit, void* __restrict__ out, int out_dt) {
    constexpr int Dh = kDecodeDh;
    const int bh = blockIdx.x;  // b*Hq + h
    const int Hq = Hk * G;
    const int b = bh / Hq, h = bh - b * Hq;
    const int hk = h / G, g = h - hk * G;
    const int d = threadIdx.x;
    const float* base = part + ((int64_t)(b * Hk + hk) * nsplit) * G * (Dh + 2) + g * (Dh + 2);
    float M = -__builtin_inff();
    for (int s = 0; s < nsplit; s++) M = fmaxf(M, base[(int64_t)s * G * (Dh + 2)]);
    float L = 0.0f, A = 0.0f;
    for (int s = 0; s < nsplit; s++) {
        const float* ps = base + (int64_t)s * G * (Dh + 2);
        if (ps[0] == -__builtin_inff()) continue;
        const float c = __expf(ps[0] - M);
        L = fmaf(ps[1], c, L);
        A = fmaf(ps[2 + d], c, A);
    }
    st_act(out, (int64_t)bh * Dh + d, A / L, out_dt);
}

// ---- elementwise -----------------------------------------------------------------
__global__ __launch_bounds__(256) void elementwise_kernel(int op, const void* __restrict__ a, int a_dt,
                                                          const void* __restrict__ b, int b_dt,
                                                          void* __restrict__ out, int out_dt, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const float x = ld_act(a, i, a_dt);
        float r;
        if (op == JH_OP_SILU) {
            r = x / (1.0f + (float)exp((double)(-x)));
        } else {
            const float y = ld_act(b, i, b_dt);
            r = op == JH_OP_ADD ? x + y : op == JH_OP_MUL ? x * y : (x / (1.0f + (float)exp((double)(-x)))) * y;
        }
        st_act(out, i, r, out_dt);
    }
}

// ---- Argmax: one block of 1024 per row; first index of the maximum ----------------
__global__ __launch_bounds__(1024) void argmax_kernel(const void* __restrict__ x, int x_dt, int64_t n,
                                                      int32_t* __restrict__ out) {
    __shared__ float bv[16];
    __shared__ int64_t bi[16];
    const int64_t r = blockIdx.x;
    float best = -__builtin_inff();
    int64_t idx = n;  // "none": loses every tie
    for (int64_t i = threadIdx.x; i < n; i += 1024) {
        const float v = ld_act(x, r * n + i, x_dt);
        if (v > best) best = v, idx = i;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o, 64);
        const int64_t oi = __shfl_xor(idx, o, 64);
        if (ov > best || (ov == best && oi < idx)) best = ov, idx = oi;
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) bv[w] = best, bi[w] = idx;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < 16; k++)
            if (bv[k] > best || (bv[k] == best && bi[k] < idx)) best = bv[k], idx = bi[k];
        out[r] = idx < n ? (int32_t)idx : 0;
    }
}

// ---- row gather and KV append ------------------------------------------------------
__global__ __launch_bounds__(256) void take_rows_kernel(const uint8_t* __restrict__ table, int64_t row_bytes,
                                                        int64_t n_rows, const int32_t* __restrict__ ids,
                                                        uint8_t* __restrict__ out) {
    const int64_t k = blockIdx.x;
    const int32_t id = ids[k];
    const bool ok = id >= 0 && id < n_rows;
    for (int64_t i = threadIdx.x; i < row_bytes; i += 256)
        out[k * row_bytes + i] = ok ? table[(int64_t)id * row_bytes + i] : (uint8_t)0;
}

__global__ __launch_bounds__(256) void kv_append_kernel(void* __restrict__ kc, void* __restrict__ vc, int c_dt,
                                                        const void* __restrict__ kn, const void* __restrict__ vn,
                                                        int n_dt, int64_t BH, int64_t cap, int64_t pos, int64_t L,
                                                        int64_t Dh) {
    const int64_t total = BH * L * Dh;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t d = t % Dh, rl = t / Dh;
        const int64_t l = rl % L, bh = rl / L;
        const int64_t dst = (bh * cap + pos + l) * Dh + d;
        st_act(kc, dst, ld_act(kn, t, n_dt), c_dt);
        st_act(vc, dst, ld_act(vn, t, n_dt), c_dt);
    }
}

unsigned grid_for(int64_t n, int64_t per_block, int64_t cap) {
    int64_t g = (n + per_block - 1) / per_block;
    if (g > cap) g = cap;
    return (unsigned)(g < 1 ? 1 : g);
}

}  // namespace

Status launch_rms_norm(const void* x, int x_dt, const void* w, int w_dt, float eps, void* out, int out_dt,
                       int64_t rows, int64_t d, hipStream_t st) {
    if (rows == 0) return Status::ok();
    if (rows > 0x7fffffff) return Status::fail(JH_ERR_UNSUPPORTED, "rms_norm: too many rows");
    hipLaunchKernelGGL(rms_norm_kernel, dim3((unsigned)rows), dim3(256), 0, st, x, x_dt, w, w_dt, eps, out, out_dt, d);
    return Status::ok();
}

Status launch_rope(const void* x, int x_dt, void* out, int out_dt, int64_t rows, int64_t L, int64_t D, int dims,
                   bool traditional, float base, float scale, int64_t offset, const float* freqs, hipStream_t st) {
    const int64_t total = rows * (D - dims / 2);
    if (total == 0) return Status::ok();
    hipLaunchKernelGGL(rope_kernel, dim3(grid_for(total, 256, 16384)), dim3(256), 0, st, x, x_dt, out, out_dt, rows,
                       L, D, dims, traditional ? 1 : 0, base, scale, offset, freqs);
    return Status::ok();
}

bool sdpa_decode_ok(int q_dt, int kv_dt, int64_t Hq, int64_t Hk, int64_t Lq, int64_t Dh) {
    const int64_t G = Hk > 0 ? Hq / Hk : 0;
    return Lq == 1 && Dh == kDecodeDh && kv_dt == JH_BF16 && (G == 1 || G == 2 || G == 4 || G == 8) &&
           (q_dt == JH_BF16 || q_dt == JH_F32);
}

int64_t sdpa_splits(int64_t B, int64_t Hk, int64_t Lk, int num_cus) {
    // about two blocks per CU, at least 64 keys per block
    int64_t n = (2 * (int64_t)num_cus + B * Hk - 1) / (B * Hk);
    const int64_t by_len = (Lk + 63) / 64;
    if (n > by_len) n = by_len;
    if (n > 65535) n = 65535;
    return n < 1 ? 1 : n;
}

size_t sdpa_workspace_bytes(int q_dt, int kv_dt, int64_t B, int64_t Hq, int64_t Hk, int64_t Lq, int64_t Lk,
                            int64_t Dh, int num_cus) {
    if (!sdpa_decode_ok(q_dt, kv_dt, Hq, Hk, Lq, Dh) || Lk <= 0) return 0;
    const int64_t G = Hq / Hk;
    const int64_t nsplit = sdpa_splits(B, Hk, Lk, num_cus);
    return sizeof(float) * (size_t)(B * Hk * nsplit * G * (kDecodeDh + 2));
}

Status launch_sdpa(const void* q, int q_dt, const void* k, const void* v, int kv_dt, void* out, int out_dt,
                   int64_t B, int64_t Hq, int64_t Hk, int64_t Lq, int64_t Lk, int64_t kcap, int64_t Dh, float scale,
                   bool causal, void* workspace, int num_cus, hipStream_t st) {
    if (B * Hq * Lq == 0) return Status::ok();
    if (sdpa_decode_ok(q_dt, kv_dt, Hq, Hk, Lq, Dh) && Lk > 0) {
        const int G = (int)(Hq / Hk);
        const int64_t nsplit = sdpa_splits(B, Hk, Lk, num_cus);
        const int kps = (int)((Lk + nsplit - 1) / nsplit);
        float* part = static_cast<float*>(workspace);
        const dim3 grid((unsigned)(B * Hk), (unsigned)nsplit);
        auto go = [&](auto kern) {
            hipLaunchKernelGGL(kern, grid, dim3(256), 0, st, q, q_dt, static_cast<const uint16_t*>(k),
                               static_cast<const uint16_t*>(v), (int)Hk, (int)Lk, (int)kcap, scale, kps, part);
        };
        if (G == 1) go(sdpa_decode_split_kernel<1>);
        else if (G == 2) go(sdpa_decode_split_kernel<2>);
        else if (G == 4) go(sdpa_decode_split_kernel<4>);
        else go(sdpa_decode_split_kernel<8>);
        hipLaunchKernelGGL(sdpa_decode_merge_kernel, dim3((unsigned)(B * Hq)), dim3(kDecodeDh), 0, st, part, (int)Hk, G,
                           (int)nsplit, out, out_dt);
        return Status::ok();
    }
    if (Dh > 256) return Status::fail(JH_ERR_UNSUPPORTED, "sdpa: head_dim above 256");
    hipLaunchKernelGGL(sdpa_rows_kernel, dim3((unsigned)(B * Hq * Lq)), dim3(256), 0, st, q, q_dt, k, v, kv_dt, out,
                       out_dt, (int)Hq, (int)Hk, (int)Lq, (int)Lk, (int)kcap, (int)Dh, scale, causal ? 1 : 0);
    return Status::ok();
}

Status launch_elementwise(int op, const void* a, int a_dt, const void* b, int b_dt, void* out, int out_dt, int64_t n,
                          hipStream_t st) {
    if (n == 0) return Status::ok();
    hipLaunchKernelGGL(elementwise_kernel, dim3(grid_for(n, 256, 16384)), dim3(256), 0, st, op, a, a_dt, b, b_dt, out,
                       out_dt, n);
    return Status::ok();
}

Status launch_argmax(const void* x, int x_dt, int64_t rows, int64_t n, int32_t* out, hipStream_t st) {
    if (rows == 0) return Status::ok();
    hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)rows), dim3(1024), 0, st, x, x_dt, n, out);
    return Status::ok();
}

Status launch_take_rows(const void* table, int64_t row_bytes, int64_t n_rows, const int32_t* ids, int64_t n_ids,
                        void* out, hipStream_t st) {
    if (n_ids == 0 || row_bytes == 0) return Status::ok();
    hipLaunchKernelGGL(take_rows_kernel, dim3((unsigned)n_ids), dim3(256), 0, st,
                       static_cast<const uint8_t*>(table), row_bytes, n_rows, ids, static_cast<uint8_t*>(out));
    return Status::ok();
}

Status launch_kv_append(void* kc, void* vc, int c_dt, const void* kn, const void* vn, int n_dt, int64_t BH,
                        int64_t cap, int64_t pos, int64_t L, int64_t Dh, hipStream_t st) {
    const int64_t total = BH * L * Dh;
    if (total == 0) return Status::ok();
    hipLaunchKernelGGL(kv_append_kernel, dim3(grid_for(total, 256, 16384)), dim3(256), 0, st, kc, vc, c_dt, kn, vn,
                       n_dt, BH, cap, pos, L, Dh);
    return Status::ok();
}

}  // namespace jh
