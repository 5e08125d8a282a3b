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
#include "qmv_tile.hpp"

namespace jh {
namespace {

__device__ __forceinline__ float ld_act(const void* p, int64_t i, int dt) {
    if (dt == JH_BF16) return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
    if (dt == JH_F16) return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
    return static_cast<const float*>(p)[i];
}

// Element i of an activation as two steps, so that a kernel can issue the load
// early and convert after later loads are in flight: ld_word reads the aligned
// 32-bit word holding the element (the element itself for f32), with no branch
// on the dtype; word_to_f32 extracts and converts it.
__device__ __forceinline__ uint32_t ld_word(const void* p, int64_t i, int dt) {
    // pointer arithmetic (not an integer round trip) keeps the load global
    const char* e = static_cast<const char*>(p) + (dt == JH_F32 ? i * 4 : i * 2);
    return *reinterpret_cast<const uint32_t*>(e - (reinterpret_cast<uintptr_t>(e) & 3));
}

__device__ __forceinline__ float word_to_f32(uint32_t w, const void* p, int64_t i, int dt) {
    if (dt == JH_F32) return __uint_as_float(w);
    const bool hi = ((reinterpret_cast<uintptr_t>(p) + (uintptr_t)(i * 2)) & 2) != 0;
    const uint16_t h = static_cast<uint16_t>(hi ? (w >> 16) : w);
    return dt == JH_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
}

__device__ __forceinline__ void st_act(void* p, int64_t i, float v, int dt) {
    if (dt == JH_BF16)
        static_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
    else if (dt == JH_F16)
        static_cast<uint16_t*>(p)[i] = f32_to_f16(v);
    else
        static_cast<float*>(p)[i] = v;
}

// A 16-byte row chunk of 8 bf16 or f16 values (a K/V cache row) as fp32.
template <bool F16>
__device__ __forceinline__ void unpack8(uint4 r, float (&f)[8]) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int q = 0; q < 4; q++) {
        if constexpr (F16) {
            f[2 * q] = f16_to_f32(static_cast<uint16_t>(w[q]));
            f[2 * q + 1] = f16_to_f32(static_cast<uint16_t>(w[q] >> 16));
        } else {
            f[2 * q] = __uint_as_float(w[q] << 16);
            f[2 * q + 1] = __uint_as_float(w[q] & 0xFFFF0000u);
        }
    }
}

// fp32 -> a cache element (bf16 or f16, nearest even) and back, for the new key
// and value of a one-token attention, which score as the values the cache holds.
template <bool F16>
__device__ __forceinline__ uint16_t to_cache(float v) {
    if constexpr (F16) return f32_to_f16(v);
    else return f32_to_bf16(v);
}
template <bool F16>
__device__ __forceinline__ float from_cache(uint16_t h) {
    if constexpr (F16) return f16_to_f32(h);
    else return bf16_to_f32(h);
}

// Sum over a block of 256 threads; every thread gets the total.
__device__ float block_sum256(float v, float* red) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    __syncthreads();
    if (l == 0) red[w] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// ---- RMSNorm -------------------------------------------------------------------
// A row's elements are loaded into registers in one burst (no load waits on an
// earlier one), squared and summed, then scaled from the registers: x is read
// once. Rows of up to 1024 take one wave each (per-head norms), longer rows one
// block of 256 threads.
template <int PER>  // elements per lane (wave kernel) or per thread (block kernel)
__device__ __forceinline__ void load_row(const void* x, int x_dt, int64_t base, int64_t d, int t, int stride,
                                         float* v) {
#pragma unroll
    for (int e = 0; e < PER; e++) {
        const int64_t i = t + (int64_t)e * stride;
        v[e] = i < d ? ld_act(x, base + i, x_dt) : 0.0f;
    }
}

template <int PER>
__global__ __launch_bounds__(256) void rms_norm_wave_kernel(const void* __restrict__ x, int x_dt,
                                                            const void* __restrict__ w, int w_dt, float eps,
                                                            void* __restrict__ out, int out_dt, int64_t rows,
                                                            int64_t d) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= rows) return;
    float v[PER];
    load_row<PER>(x, x_dt, r * d, d, lane, 64, v);
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < PER; e++) ss = fmaf(v[e], v[e], ss);
    ss = wave_sum(ss);
    const float inv = 1.0f / (float)sqrt((double)(ss / (float)d + eps));
#pragma unroll
    for (int e = 0; e < PER; e++) {
        const int64_t i = lane + (int64_t)e * 64;
        if (i < d) st_act(out, r * d + i, (v[e] * inv) * ld_act(w, i, w_dt), out_dt);
    }
}

template <int PER>
__global__ __launch_bounds__(256) void rms_norm_block_kernel(const void* __restrict__ x, int x_dt,
                                                             const void* __restrict__ w, int w_dt, float eps,
                                                             void* __restrict__ out, int out_dt, int64_t d) {
    __shared__ float red[4];
    const int64_t r = blockIdx.x;
    float v[PER];
    load_row<PER>(x, x_dt, r * d, d, threadIdx.x, 256, v);
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < PER; e++) ss = fmaf(v[e], v[e], ss);
    ss = block_sum256(ss, red);
    const float inv = 1.0f / (float)sqrt((double)(ss / (float)d + eps));
#pragma unroll
    for (int e = 0; e < PER; e++) {
        const int64_t i = threadIdx.x + (int64_t)e * 256;
        if (i < d) st_act(out, r * d + i, (v[e] * inv) * ld_act(w, i, w_dt), out_dt);
    }
}

// Rows longer than 256 * 64 elements: two passes over x.
__global__ __launch_bounds__(256) void rms_norm_long_kernel(const void* __restrict__ x, int x_dt,
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
    for (int64_t i = threadIdx.x; i < d; i += 256)
        st_act(out, r * d + i, (ld_act(x, r * d + i, x_dt) * inv) * ld_act(w, i, w_dt), out_dt);
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

// cos and sin of the RoPE angles at one position: out[i] = cos(theta_i),
// out[dims/2 + i] = sin(theta_i), theta_i = pos * scale * inv_i with the same
// inv_i and double evaluation as rope_kernel. Kernels that rotate many heads at
// one position read these instead of each evaluating pow/cos/sin in double.
__global__ __launch_bounds__(64) void rope_table_kernel(int dims, float base, float scale, int64_t pos,
                                                         const float* __restrict__ freqs, float* __restrict__ out) {
    const int half = dims / 2;
    for (int i = threadIdx.x; i < half; i += 64) {
        const float inv = freqs ? 1.0f / freqs[i] : (float)pow((double)base, -(double)(2 * i) / (double)dims);
        const float theta = (float)pos * scale * inv;
        out[i] = (float)cos((double)theta);
        out[half + i] = (float)sin((double)theta);
    }
}

// ---- the two halves of a split RMSNorm ---------------------------------------------
// Producer half for one row of d: out = bf16(x * w); block b sums x^2 over its
// 2048 elements into stats[b] (its 8 loads per thread issue together), block 0
// zeroes the slots past the grid. Consumer half (the fallback of a product that
// cannot apply the statistics in its epilogue): out = bf16(u / sqrt(sum(stats) /
// d + eps)).
constexpr int kPrepPer = 8;  // elements per thread of norm_prepare_kernel

__global__ __launch_bounds__(256) void norm_prepare_kernel(const void* __restrict__ x, int x_dt, int64_t d,
                                                           const void* __restrict__ w, int w_dt,
                                                           uint16_t* __restrict__ out, float* __restrict__ stats) {
    __shared__ float red[4];
    const int64_t base = (int64_t)blockIdx.x * 256 * kPrepPer + threadIdx.x;
    float xv[kPrepPer], wv[kPrepPer];
#pragma unroll
    for (int e = 0; e < kPrepPer; e++) {
        const int64_t i = base + 256 * e;
        xv[e] = i < d ? ld_act(x, i, x_dt) : 0.0f;
        wv[e] = i < d ? ld_act(w, i, w_dt) : 0.0f;
    }
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < kPrepPer; e++) {
        const int64_t i = base + 256 * e;
        ss = fmaf(xv[e], xv[e], ss);
        if (i < d) out[i] = f32_to_bf16(xv[e] * wv[e]);
    }
    ss = block_sum256(ss, red);
    if (threadIdx.x == 0) stats[blockIdx.x] = ss;
    if (blockIdx.x == 0)
        for (int i = gridDim.x + threadIdx.x; i < kNormSlots; i += 256) stats[i] = 0.0f;
}

// The decode step's first launch: the embedding row of token ids[0] (Dequantize
// of the row TakeAxis picks, qwen/embed.go:78-83, zero for an id outside the
// table, as take_rows gives), the first block's split RMSNorm producer half on
// it, and, from one more block when cs is given, the RoPE factor table at pos.
// Blocks below nb follow norm_prepare_kernel element for element: h is the
// value Dequantize stores, the sums of squares run in the same order, so u and
// the statistics are those of the three separate launches bit for bit.
template <int BITS>
__global__ __launch_bounds__(256) void embed_norm_kernel(const int32_t* __restrict__ ids, const uint32_t* __restrict__ W,
                                                         const void* __restrict__ S, const void* __restrict__ B,
                                                         int sb_dt, int64_t vocab, int64_t d, int gs,
                                                         const void* __restrict__ w, int w_dt, float* __restrict__ h,
                                                         uint16_t* __restrict__ out, float* __restrict__ stats, int nb,
                                                         int rope_dims, float base, float scale, int64_t pos,
                                                         float* __restrict__ cs) {
    constexpr int VPW = 32 / BITS;
    constexpr uint32_t MASK = (1u << BITS) - 1u;
    if ((int)blockIdx.x >= nb) {  // the RoPE table, as rope_table_kernel
        const int half = rope_dims / 2;
        for (int i = threadIdx.x; i < half; i += 256) {
            const float inv = (float)pow((double)base, -(double)(2 * i) / (double)rope_dims);
            const float theta = (float)pos * scale * inv;
            cs[i] = (float)cos((double)theta);
            cs[half + i] = (float)sin((double)theta);
        }
        return;
    }
    __shared__ float red[4];
    const int32_t id = ids[0];
    const bool ok = id >= 0 && id < vocab;
    const int64_t P = d / VPW, G = d / gs;
    const int64_t row = ok ? (int64_t)id : 0;
    const int64_t base_i = (int64_t)blockIdx.x * 256 * kPrepPer + threadIdx.x;
    float xv[kPrepPer], wv[kPrepPer];
#pragma unroll
    for (int e = 0; e < kPrepPer; e++) {
        const int64_t i = base_i + 256 * e;
        float v = 0.0f;
        if (i < d && ok) {
            const uint32_t word = W[row * P + i / VPW];
            const int64_t g = i / gs;
            v = unfused_qsb((float)((word >> (BITS * (int)(i % VPW))) & MASK), load_sb(S, row * G + g, sb_dt),
                            load_sb(B, row * G + g, sb_dt));
        }
        xv[e] = v;
        wv[e] = i < d ? ld_act(w, i, w_dt) : 0.0f;
    }
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < kPrepPer; e++) {
        const int64_t i = base_i + 256 * e;
        ss = fmaf(xv[e], xv[e], ss);
        if (i < d) {
            h[i] = xv[e];
            out[i] = f32_to_bf16(xv[e] * wv[e]);
        }
    }
    ss = block_sum256(ss, red);
    if (threadIdx.x == 0) stats[blockIdx.x] = ss;
    if (blockIdx.x == 0)
        for (int i = nb + threadIdx.x; i < kNormSlots; i += 256) stats[i] = 0.0f;
}

__global__ __launch_bounds__(256) void norm_apply_kernel(const uint16_t* __restrict__ u, int64_t d,
                                                         const float* __restrict__ stats, float eps,
                                                         uint16_t* __restrict__ out) {
    __shared__ float red[4];
    float t = 0.0f;
    for (int i = threadIdx.x; i < kNormSlots; i += 256) t += stats[i];
    t = block_sum256(t, red);
    const float inv = 1.0f / (float)sqrt((double)(t / (float)d + eps));
    for (int64_t i = threadIdx.x; i < d; i += 256) out[i] = f32_to_bf16(bf16_to_f32(u[i]) * inv);
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
    mx = wave_max(mx);
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
constexpr int kDecodeDh = 128;


template <int G, bool KF16>
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
    // the next key's rows are loaded before this key is scored
    int j = j_begin + wave * 4 + kg;
    uint4 kn = make_uint4(0, 0, 0, 0), vn = kn;
    if (j < j_end) {
        kn = *reinterpret_cast<const uint4*>(k + kbase + (int64_t)j * Dh + 8 * kl);
        vn = *reinterpret_cast<const uint4*>(v + kbase + (int64_t)j * Dh + 8 * kl);
    }
    for (; j < j_end; j += 16) {
        const uint4 kr = kn, vr = vn;
        if (j + 16 < j_end) {
            kn = *reinterpret_cast<const uint4*>(k + kbase + (int64_t)(j + 16) * Dh + 8 * kl);
            vn = *reinterpret_cast<const uint4*>(v + kbase + (int64_t)(j + 16) * Dh + 8 * kl);
        }
        float kf[8], vf[8];
        unpack8<KF16>(kr, kf);
        unpack8<KF16>(vr, vf);
#pragma unroll
        for (int g = 0; g < G; g++) {
            float s = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; e++) s = fmaf(qv[g][e], kf[e], s);
            s = row16_sum(s);
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

// Merge the splits of one (b, query head): blockDim / 128 groups (1 to 4, one
// per 16 splits) of 128 threads each take a share of the splits (thread d of a
// group owns feature d), reading them 16 at a time with each chunk's loads
// issued together and folding them in with an online rescale; the groups meet
// in LDS. Up to 64 splits cost one memory round trip.
constexpr int kMaxSplits = 1024;
constexpr int kMergeGroups = 4;
int merge_groups(int64_t nsplit) { return (int)std::min<int64_t>(kMergeGroups, (nsplit + 15) / 16); }

__global__ __launch_bounds__(128 * kMergeGroups) void sdpa_decode_merge_kernel(const float* __restrict__ part, int Hk,
                                                                               int G, int nsplit,
                                                                               void* __restrict__ out, int out_dt) {
    constexpr int Dh = kDecodeDh, C = 16;
    const int bh = blockIdx.x;  // b*Hq + h
    const int Hq = Hk * G;
    const int b = bh / Hq, h = bh - b * Hq;
    const int hk = h / G, g = h - hk * G;
    const int d = threadIdx.x & (Dh - 1), grp = threadIdx.x / Dh, ng = blockDim.x / Dh;
    const int64_t stride = (int64_t)G * (Dh + 2);
    const float* base = part + ((int64_t)(b * Hk + hk) * nsplit) * stride + g * (Dh + 2);
    const int per = (nsplit + ng - 1) / ng;
    const int s_begin = grp * per, s_end = min(nsplit, s_begin + per);
    float M = -__builtin_inff(), L = 0.0f, A = 0.0f;
    for (int s0 = s_begin; s0 < s_end; s0 += C) {
        float mv[C], lv[C], av[C];
#pragma unroll
        for (int u = 0; u < C; u++) {
            const bool in = s0 + u < s_end;
            const float* ps = base + (int64_t)(in ? s0 + u : s_end - 1) * stride;  // in bounds either way
            mv[u] = in ? ps[0] : -__builtin_inff();
            lv[u] = in ? ps[1] : 0.0f;
            av[u] = in ? ps[2 + d] : 0.0f;
        }
        float mn = M;
#pragma unroll
        for (int u = 0; u < C; u++) mn = fmaxf(mn, mv[u]);
        if (mn == -__builtin_inff()) continue;  // no keys so far
        const float corr = __expf(M - mn);
        L *= corr;
        A *= corr;
#pragma unroll
        for (int u = 0; u < C; u++) {
            const float c = __expf(mv[u] - mn);
            L = fmaf(lv[u], c, L);
            A = fmaf(av[u], c, A);
        }
        M = mn;
    }
    if (ng == 1) {
        st_act(out, (int64_t)bh * Dh + d, A / L, out_dt);
        return;
    }
    __shared__ float gm[kMergeGroups], gl[kMergeGroups], ga[kMergeGroups][Dh];
    if (d == 0) gm[grp] = M, gl[grp] = L;
    ga[grp][d] = A;
    __syncthreads();
    if (grp != 0) return;
    float Mt = gm[0];
    for (int q = 1; q < ng; q++) Mt = fmaxf(Mt, gm[q]);
    float Lt = 0.0f, At = 0.0f;
    for (int q = 0; q < ng; q++) {
        const float c = gm[q] == -__builtin_inff() ? 0.0f : __expf(gm[q] - Mt);
        Lt = fmaf(gl[q], c, Lt);
        At = fmaf(ga[q][d], c, At);
    }
    st_act(out, (int64_t)bh * Dh + d, At / Lt, out_dt);
}

// Per-head RMSNorm of one 128-feature head held as lane i: (a, b) = features
// (i, i + 64) of a wave, with the lane's weights (w0, w1) = (w[i], w[i + 64]).
// Contraction into FMAs is off in these helpers: the kernels that share them
// (the standalone q/k norm + RoPE + append, the one-launch attention) then store
// the same bits for a new key, which an f16 cache keeps to 11 bits.
__device__ __forceinline__ void head_rms_norm_w(float& a, float& b, float w0, float w1, float eps) {
#pragma clang fp contract(off)
    const float ss = wave_sum(fmaf(a, a, b * b));
    const float inv = 1.0f / (float)sqrt((double)(ss / 128.0f + eps));
    a = (a * inv) * w0;
    b = (b * inv) * w1;
}

// w == nullptr skips the norm (heads without QNorm/KNorm).
__device__ __forceinline__ void head_rms_norm(float& a, float& b, const void* w, int w_dt, float eps, int i) {
    if (!w) return;
    head_rms_norm_w(a, b, ld_act(w, i, w_dt), ld_act(w, i + 64, w_dt), eps);
}

// Non-traditional RoPE factors of the pair (i, i + 64) of a 128-feature head at
// `pos`: angle pos * scale * base^(-2i/128), cos/sin/pow in double.
__device__ __forceinline__ void head_rope_factors(float base, float scale, int64_t pos, int i, float& c, float& sn) {
    const float fi = (float)pow((double)base, -(double)(2 * i) / 128.0);
    const float theta = (float)pos * scale * fi;
    c = (float)cos((double)theta);
    sn = (float)sin((double)theta);
}

__device__ __forceinline__ void rotate_pair(float& a, float& b, float c, float sn) {
#pragma clang fp contract(off)
    const float ra = a * c - b * sn, rb = a * sn + b * c;
    a = ra;
    b = rb;
}

// With `cs` (rope_table_kernel's output for this position) the factors are read.
__device__ __forceinline__ void head_rope(float& a, float& b, float base, float scale, int64_t pos, int i,
                                          const float* cs = nullptr) {
    float c, sn;
    if (cs) {
        c = cs[i];
        sn = cs[64 + i];
    } else {
        head_rope_factors(base, scale, pos, i, c, sn);
    }
    rotate_pair(a, b, c, sn);
}

// ---- Qwen3 attention prologue: per-head q/k RMSNorm, RoPE, KV append ------------
// One wave per head of one token's q/k/v vector [(Hq + 2Hk) * 128]: query heads
// are normalised with q_norm and rotated into q_out; key heads normalised with
// k_norm, rotated and written to row `pos` of the key cache; value heads copied
// to the value cache. head_dim 128, non-traditional RoPE: lane i holds features
// i and i + 64, which is exactly one rotated pair, so the rotation is lane-local.
// (qwen/attention.go:101-122: QNorm/KNorm.Forward, RoPE, KVCache.Update.)
__global__ __launch_bounds__(256) void qk_norm_rope_append_kernel(
    const void* __restrict__ qkv, int qkv_dt, int Hq, int Hk, const void* __restrict__ qn_w,
    const void* __restrict__ kn_w, int w_dt, float eps, float base, float scale, int64_t pos,
    void* __restrict__ kc, void* __restrict__ vc, int c_dt, int64_t cap, void* __restrict__ q_out, int q_dt) {
    constexpr int Dh = 128, half = 64;
    const int head = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int i = threadIdx.x & 63;
    if (head >= Hq + 2 * Hk) return;
    const int64_t o = (int64_t)head * Dh;
    float a = ld_act(qkv, o + i, qkv_dt), b = ld_act(qkv, o + i + half, qkv_dt);
    if (head >= Hq + Hk) {  // value head: to the cache as is
        const int64_t dst = ((int64_t)(head - Hq - Hk) * cap + pos) * Dh;
        st_act(vc, dst + i, a, c_dt);
        st_act(vc, dst + i + half, b, c_dt);
        return;
    }
    const bool is_q = head < Hq;
    head_rms_norm(a, b, is_q ? qn_w : kn_w, w_dt, eps, i);
    head_rope(a, b, base, scale, pos, i);
    const float ra = a, rb = b;
    if (is_q) {
        st_act(q_out, o + i, ra, q_dt);
        st_act(q_out, o + i + half, rb, q_dt);
    } else {
        const int64_t dst = ((int64_t)(head - Hq) * cap + pos) * Dh;
        st_act(kc, dst + i, ra, c_dt);
        st_act(kc, dst + i + half, rb, c_dt);
    }
}

// ---- one-token attention in one launch ---------------------------------------------
// Attention.ForwardCached for one new token (qwen/attention.go:98-128) after the
// q/k/v product: per-head q/k RMSNorm and RoPE, the KV-cache append, and SDPA
// over keys 0..pos. The pos cache rows are split evenly over blocks (split, hk),
// kps rows each, for the G = Hq/Hk query heads of kv head hk; the new key at pos
// has a block of its own (split 0) when the grid has room, else it joins the
// last split:
//   1. its K/V rows are requested first (they do not depend on q), then every
//      block normalises and rotates its G query heads into LDS (a few hundred
//      flops, cheaper than a launch); the new key's block normalises and
//      rotates it, writes the new key and value rows to the caches, and scores
//      them from LDS (bf16-rounded, as the cache holds them), never reading row
//      pos back;
//   2. 16 key slots per block (4 per wave, a 16-lane row per key, 8 features per
//      lane) run an online softmax over the slot's keys, U keys per load batch;
//   3. the slots merge in registers (cross-row permlane swaps) and then across
//      the 4 waves in LDS;
//   4. with one split the block writes the output; otherwise (max, sum,
//      weighted values) go to the workspace and are merged in split order,
//      either
//      - in the same launch (`sync` set, kv heads a multiple of 8): the grid
//        is 1-D and block b runs on XCD b % 8 (workgroups are dealt to the 8
//        XCDs round-robin in launch order; jh_create checks this on the
//        device and leaves `sync` unset otherwise), so every split of kv head
//        hk runs on XCD hk % 8 and shares its L2. Each block stores its
//        partials (128-byte-aligned records, plain stores: the per-CU L1 is
//        write-through), waits for the stores, and adds one to the head's
//        arrival counter with an L2 atomic; the block that arrives last reads
//        the partials back from that L2 and writes the output, then clears
//        the counter for the next call. Nothing leaves the XCD: no release to
//        memory, no second launch. (The same protocol at agent scope -- stores
//        written through to memory, memory atomics, 9.7 against 9.1 us per
//        layer at 512 keys -- lost to the merge launch, and an agent-scope
//        release per block, an L2 writeback, cost ten times it.)
//      - or in sdpa_decode_merge_kernel, from sdpa_decode_split_kernel's
//        layout.
struct AttnArgs {
    const void* qkv;    // [(Hq + 2 Hk) * 128]: q heads, k heads, v heads
    int qkv_dt;
    const void* qn_w;   // [128] or nullptr
    const void* kn_w;
    int w_dt;
    float eps, base, rscale, scale;
    const float* rope_cs;  // [128]: cos, sin at pos (rope_table_kernel), or nullptr
    int64_t pos;
    uint16_t* kc;       // bf16 or f16 [Hk, cap, 128]
    uint16_t* vc;
    int64_t cap;
    int Hk, nsplit, kps;
    int owner_alone;    // 1: split 0 takes only the new key; 0: the last split also takes it
    float* part;        // [Hk, nsplit, G, 130], or [Hk, nsplit] records of attn_rec_floats(G) with `sync`
    void* out;          // [Hq * 128]
    int out_dt;
    int* sync;          // [Hk] arrival counters (zero between calls), or nullptr: merge launch
    int* flags;         // fused q/k/v + attention launch: this XCD's arrival flags, cleared by its
                        // last attention block; nullptr otherwise
    int nflags;
    int* marker;        // fused launch: this XCD's give-up marker (set when a wait gave up; stays set
                        // until the host resets it), nullptr otherwise
};

// Floats of one split's partials in the in-launch merge layout: G x (max, sum,
// 128 values), rounded up to whole 128-byte lines so that no two blocks' records
// share a cache line.
constexpr int attn_rec_floats(int G) { return (G * (kDecodeDh + 2) + 31) / 32 * 32; }
static_assert(kDecodeDh == 128, "the in-launch merge maps 64 lanes onto G x 128 outputs");

// One block's share of a one-token attention: split `split` of kv head hk.
// FUSED (the q/k/v product ran earlier in the same launch, on this XCD): the
// block's K/V rows are requested first, then wait() returns once the product's
// rows are all stored (false) or once it gave up (true), and q/k/v are read
// device-coherently from the L2. When a wait of the XCD gave up (now or in an
// earlier call the host has not reset), the head's output is NaN and the flags
// are left as they are for the host to reset.
template <int G, int U, bool FUSED, bool KF16, class Wait>  // U: keys per slot per load batch; KF16: f16 caches
__device__ __forceinline__ void attn_body(const AttnArgs& a, const int split, const int hk, Wait wait) {
    constexpr int Dh = 128;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int kg = lane >> 4, kl = lane & 15;
    const int Hq = a.Hk * G;
    // the cache rows 0..pos-1 split evenly; the new key has a block of its own
    // (split 0, dispatched first) or joins the last split
    const bool owner = a.owner_alone ? split == 0 : split == a.nsplit - 1;
    const int64_t cs = a.owner_alone ? (int64_t)split - 1 : split;  // -1: the new key's own block
    const int64_t j_begin = cs < 0 ? 0 : cs * a.kps;
    const int64_t jc_end = cs < 0 ? 0 : min(a.pos, j_begin + a.kps);  // cache rows scored by this block
    // This block's cache rows as buffer resources over rows [0, jc_end) of the
    // head: a row past jc_end reads as zeros, with no branch around the load.
    const __amdgpu_buffer_rsrc_t kb = make_rsrc(a.kc + (int64_t)hk * a.cap * Dh, (uint32_t)(jc_end * Dh * 2));
    const __amdgpu_buffer_rsrc_t vb = make_rsrc(a.vc + (int64_t)hk * a.cap * Dh, (uint32_t)(jc_end * Dh * 2));
    const int slot = wave * 4 + kg;

    // 1. The prologue's inputs (this wave's query heads, the norm weights, the
    // RoPE factors; the new key and value in the new key's block) are requested
    // first and the block's K/V rows after them: loads complete in order, so the
    // prologue waits for its own inputs alone while the K/V rows stream in.
    constexpr int QPW = (G + 3) / 4;  // query heads per wave
    const bool qn = a.qn_w != nullptr, kn = a.kn_w != nullptr, table = a.rope_cs != nullptr;
    const bool kv_wave = owner && wave == 3;
    // Absent inputs read a valid stand-in (the qkv row) and are replaced after.
    const void* qwp = qn ? a.qn_w : a.qkv;
    const void* kwp = kn ? a.kn_w : a.qkv;
    const float* csp = table ? a.rope_cs : static_cast<const float*>(a.qkv);
    const int qw_dt = qn ? a.w_dt : a.qkv_dt, kw_dt = kn ? a.w_dt : a.qkv_dt;
    uint4 kr[U], vr[U];  // raw bf16 rows, unpacked one key at a time
    auto load_rows = [&](uint4 (&r)[U], __amdgpu_buffer_rsrc_t src, int64_t j0) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(src, (uint32_t)((j0 + 16 * u) * Dh * 2 + 16 * kl), 0, 0);
            r[u] = make_uint4(v.x, v.y, v.z, v.w);
        }
    };
    int64_t j0 = j_begin + slot;
    bool gave_up = false;
    if constexpr (FUSED) {
        // the K/V rows do not depend on the product: in flight while it finishes
        load_rows(kr, kb, j0);
        load_rows(vr, vb, j0);
        gave_up = wait();
    }
    // q/k/v words (FUSED: bf16 or f32, stored by other CUs of this XCD, read from L2)
    const bool qf32 = a.qkv_dt == JH_F32;
    const auto rq = make_rsrc(a.qkv, (uint32_t)((Hq + 2 * a.Hk) * Dh * (qf32 ? 4 : 2)));
    auto ldq = [&](int64_t i) -> uint32_t {
        if constexpr (FUSED)
            return __builtin_amdgcn_raw_buffer_load_b32(rq, (uint32_t)(qf32 ? i : i >> 1) * 4, 0, kAuxSc1);
        else
            return ld_word(a.qkv, i, a.qkv_dt);
    };
    uint32_t qraw[QPW][2], kvraw[6], wraw[2];
#pragma unroll
    for (int i = 0; i < QPW; i++) {
        const int g = min(wave + 4 * i, G - 1);
        const int64_t o = (int64_t)(hk * G + g) * Dh;
        qraw[i][0] = ldq(o + lane);
        qraw[i][1] = ldq(o + lane + 64);
    }
    wraw[0] = ld_word(qwp, lane, qw_dt);
    wraw[1] = ld_word(qwp, lane + 64, qw_dt);
    const float rc_raw = csp[lane], rs_raw = csp[64 + lane];
    // Every wave issues the new key's loads (the same addresses in all blocks);
    // only the owner's wave 3 uses them.
    const int64_t ok = (int64_t)(Hq + hk) * Dh, ov = (int64_t)(Hq + a.Hk + hk) * Dh;
    kvraw[0] = ldq(ok + lane);
    kvraw[1] = ldq(ok + lane + 64);
    kvraw[2] = ldq(ov + lane);
    kvraw[3] = ldq(ov + lane + 64);
    kvraw[4] = ld_word(kwp, lane, kw_dt);
    kvraw[5] = ld_word(kwp, lane + 64, kw_dt);
    if constexpr (!FUSED) {
        load_rows(kr, kb, j0);
        load_rows(vr, vb, j0);
    }

    float rc = rc_raw, rsn = rs_raw;
    if (!table) head_rope_factors(a.base, a.rscale, a.pos, lane, rc, rsn);
    const float qw0 = qn ? word_to_f32(wraw[0], qwp, lane, qw_dt) : 1.0f;
    const float qw1 = qn ? word_to_f32(wraw[1], qwp, lane + 64, qw_dt) : 1.0f;
    __shared__ float q_s[G][Dh];
    __shared__ float kn_s[Dh], vn_s[Dh];
#pragma unroll
    for (int i = 0; i < QPW; i++) {
        const int g = wave + 4 * i;
        if (g >= G) break;
        const int64_t o = (int64_t)(hk * G + g) * Dh;
        float x0 = word_to_f32(qraw[i][0], a.qkv, o + lane, a.qkv_dt);
        float x1 = word_to_f32(qraw[i][1], a.qkv, o + lane + 64, a.qkv_dt);
        if (qn) head_rms_norm_w(x0, x1, qw0, qw1, a.eps);
        rotate_pair(x0, x1, rc, rsn);
        q_s[g][lane] = x0 * a.scale;
        q_s[g][lane + 64] = x1 * a.scale;
    }
    if (kv_wave) {
        float k0 = word_to_f32(kvraw[0], a.qkv, ok + lane, a.qkv_dt);
        float k1 = word_to_f32(kvraw[1], a.qkv, ok + lane + 64, a.qkv_dt);
        const float v0 = word_to_f32(kvraw[2], a.qkv, ov + lane, a.qkv_dt);
        const float v1 = word_to_f32(kvraw[3], a.qkv, ov + lane + 64, a.qkv_dt);
        if (kn) head_rms_norm_w(k0, k1, word_to_f32(kvraw[4], kwp, lane, kw_dt),
                                word_to_f32(kvraw[5], kwp, lane + 64, kw_dt), a.eps);
        rotate_pair(k0, k1, rc, rsn);
        const uint16_t bk0 = to_cache<KF16>(k0), bk1 = to_cache<KF16>(k1);
        const uint16_t bv0 = to_cache<KF16>(v0), bv1 = to_cache<KF16>(v1);
        const int64_t row = ((int64_t)hk * a.cap + a.pos) * Dh;
        a.kc[row + lane] = bk0;
        a.kc[row + lane + 64] = bk1;
        a.vc[row + lane] = bv0;
        a.vc[row + lane + 64] = bv1;
        kn_s[lane] = from_cache<KF16>(bk0);
        kn_s[lane + 64] = from_cache<KF16>(bk1);
        vn_s[lane] = from_cache<KF16>(bv0);
        vn_s[lane + 64] = from_cache<KF16>(bv1);
    }
    __syncthreads();

    // 2. online softmax over this slot's keys
    float qv[G][8];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < 8; e++) qv[g][e] = q_s[g][8 * kl + e];
    float m[G], l[G], acc[G][8];
#pragma unroll
    for (int g = 0; g < G; g++) {
        m[g] = -__builtin_inff();
        l[g] = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) acc[g][e] = 0.0f;
    }
    // Scores for the batch (keys unpacked one at a time), then the next batch's
    // keys are requested while the softmax and the value sums run, and its
    // values once those are done.
    for (; j0 < jc_end; j0 += 16 * U) {
        const bool more = j0 + 16 * U < jc_end;
        float s[G][U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            float kf[8];
            unpack8<KF16>(kr[u], kf);
            const bool in = j0 + 16 * u < jc_end;
#pragma unroll
            for (int g = 0; g < G; g++) {
                float d = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; e++) d = fmaf(qv[g][e], kf[e], d);
                d = row16_sum(d);
                s[g][u] = in ? d : -__builtin_inff();
            }
        }
        if (more) load_rows(kr, kb, j0 + 16 * U);
#pragma unroll
        for (int g = 0; g < G; g++) {
            float mn = m[g];
#pragma unroll
            for (int u = 0; u < U; u++) mn = fmaxf(mn, s[g][u]);
            // key u = 0 is always in range, so mn is finite here
            const float corr = __expf(m[g] - mn);
            l[g] *= corr;
#pragma unroll
            for (int e = 0; e < 8; e++) acc[g][e] *= corr;
#pragma unroll
            for (int u = 0; u < U; u++) {
                s[g][u] = __expf(s[g][u] - mn);
                l[g] += s[g][u];
            }
            m[g] = mn;
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            float vf[8];
            unpack8<KF16>(vr[u], vf);
#pragma unroll
            for (int g = 0; g < G; g++)
#pragma unroll
                for (int e = 0; e < 8; e++) acc[g][e] = fmaf(s[g][u], vf[e], acc[g][e]);
        }
        if (more) load_rows(vr, vb, j0 + 16 * U);
    }
    if (owner && slot == 0) {  // the new key, from LDS
        float kf[8], vf[8];
#pragma unroll
        for (int e = 0; e < 8; e++) kf[e] = kn_s[8 * kl + e], vf[e] = vn_s[8 * kl + e];
#pragma unroll
        for (int g = 0; g < G; g++) {
            float d = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; e++) d = fmaf(qv[g][e], kf[e], d);
            d = row16_sum(d);
            const float mn = fmaxf(m[g], d);
            const float corr = __expf(m[g] - mn), p = __expf(d - mn);
            l[g] = fmaf(l[g], corr, p);
#pragma unroll
            for (int e = 0; e < 8; e++) acc[g][e] = fmaf(acc[g][e], corr, p * vf[e]);
            m[g] = mn;
        }
    }

    // 3. merge the wave's 4 slots (rows of 16 lanes, permlane swaps), then the 4 waves
    __shared__ float wm[4][G], wl[4][G], wacc[4][G][Dh];
#pragma unroll
    for (int g = 0; g < G; g++) {
        const float M = rows4_max(m[g]);
        const float c = m[g] == -__builtin_inff() ? 0.0f : __expf(m[g] - M);
        const float L = rows4_sum(l[g] * c);
#pragma unroll
        for (int e = 0; e < 8; e++) acc[g][e] = rows4_sum(acc[g][e] * c);
        if (kg == 0) {
#pragma unroll
            for (int e = 0; e < 8; e++) wacc[wave][g][8 * kl + e] = acc[g][e];
            if (kl == 0) wm[wave][g] = M, wl[wave][g] = L;
        }
    }
    __syncthreads();
    constexpr int PER = (G * Dh + 255) / 256;  // outputs per thread
    float rM[PER], rL[PER], rA[PER];
#pragma unroll
    for (int r = 0; r < PER; r++) {
        const int t = threadIdx.x + 256 * r;
        rM[r] = -__builtin_inff(), rL[r] = 0.0f, rA[r] = 0.0f;
        if (t < G * Dh) {
            const int g = t / Dh, d = t - g * Dh;
            float M = wm[0][g];
#pragma unroll
            for (int w = 1; w < 4; w++) M = fmaxf(M, wm[w][g]);
            float L = 0.0f, A = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const float c = wm[w][g] == -__builtin_inff() ? 0.0f : __expf(wm[w][g] - M);
                L = fmaf(wl[w][g], c, L);
                A = fmaf(wacc[w][g][d], c, A);
            }
            rM[r] = M, rL[r] = L, rA[r] = A;
        }
    }
    if (a.nsplit == 1) {
#pragma unroll
        for (int r = 0; r < PER; r++) {
            const int t = threadIdx.x + 256 * r;
            if (t < G * Dh)
                st_act(a.out, (int64_t)hk * G * Dh + t, gave_up ? __builtin_nanf("") : rA[r] / rL[r], a.out_dt);
        }
        // the XCD's only attention block: every block has arrived (its wait saw
        // every flag set), the call is over
        if (FUSED && !gave_up)
            for (int i = threadIdx.x; i < a.nflags; i += 256) a.flags[i] = 0;
        return;
    }

    // 4. partials out
    constexpr int PS = Dh + 2;
    if (!a.sync) {
        float* mine = a.part + ((int64_t)hk * a.nsplit + split) * G * PS;
#pragma unroll
        for (int r = 0; r < PER; r++) {
            const int t = threadIdx.x + 256 * r;
            if (t < G * Dh) {
                const int g = t / Dh, d = t - g * Dh;
                mine[g * PS + 2 + d] = rA[r];
                if (d == 0) mine[g * PS] = rM[r], mine[g * PS + 1] = rL[r];
            }
        }
        return;
    }
    // in-launch layout: a record of REC floats per split, values [G][128]
    // first (16-byte aligned), then max[G], sum[G]
    constexpr int REC = attn_rec_floats(G);
    float* mine = a.part + ((int64_t)hk * a.nsplit + split) * REC;
#pragma unroll
    for (int r = 0; r < PER; r++) {
        const int t = threadIdx.x + 256 * r;
        if (t < G * Dh) {
            mine[t] = rA[r];
            if ((t & (Dh - 1)) == 0) mine[G * Dh + t / Dh] = rM[r], mine[G * Dh + G + t / Dh] = rL[r];
        }
    }

    // 5. in-launch merge on this XCD: every wave's partial stores have reached
    // the L2 before the block's arrival is counted there
    __shared__ int last;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
        last = __hip_atomic_fetch_add(a.sync + hk, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               a.nsplit - 1;
    __syncthreads();
    if (!last) return;
    // The last block: all splits' records are in this XCD's L2. Wave w merges
    // splits w, w + 4, ... in that order, SB splits per round trip, lane l holding VPL consecutive
    // outputs of one query head; the 4 waves' results meet in LDS.
    constexpr int VPL = G * Dh / 64, SB = VPL >= 16 ? 4 : (VPL >= 8 ? 8 : 16);
    const int o0 = lane * VPL, gl = o0 / Dh;
    // Reads are device-coherent (sc1): they miss this CU's L1, which could hold a
    // stale copy of a line another CU wrote, and are served by the shared L2.
    const auto hb = make_rsrc(a.part + (int64_t)hk * a.nsplit * REC, (uint32_t)(a.nsplit * REC * 4));
    // whether any wait of this XCD gave up: its marker was stored before that
    // block's arrival, so it is in the L2 by now (read with the partials)
    const int marked = FUSED ? __hip_atomic_load(a.marker, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
    float M = -__builtin_inff(), L = 0.0f, A[VPL];
#pragma unroll
    for (int e = 0; e < VPL; e++) A[e] = 0.0f;
    for (int s0 = wave; s0 < a.nsplit; s0 += 4 * SB) {
        float mv[SB], lv[SB], av[SB][VPL];
#pragma unroll
        for (int u = 0; u < SB; u++) {
            const int sp = s0 + 4 * u;
            const uint32_t rec = (uint32_t)min(sp, a.nsplit - 1) * REC * 4;  // in bounds either way
            const bool in = sp < a.nsplit;
            const float m_ = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(hb, rec + (G * Dh + gl) * 4, 0, kAuxSc1));
            mv[u] = in ? m_ : -__builtin_inff();
            lv[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(hb, rec + (G * Dh + G + gl) * 4, 0, kAuxSc1));
            if constexpr (VPL >= 4) {
#pragma unroll
                for (int e = 0; e < VPL; e += 4) {
                    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(hb, rec + (o0 + e) * 4, 0, kAuxSc1);
                    av[u][e] = __uint_as_float(v.x), av[u][e + 1] = __uint_as_float(v.y);
                    av[u][e + 2] = __uint_as_float(v.z), av[u][e + 3] = __uint_as_float(v.w);
                }
            } else {
#pragma unroll
                for (int e = 0; e < VPL; e++)
                    av[u][e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(hb, rec + (o0 + e) * 4, 0, kAuxSc1));
            }
        }
        float mn = M;
#pragma unroll
        for (int u = 0; u < SB; u++) mn = fmaxf(mn, mv[u]);
        if (mn == -__builtin_inff()) continue;  // no keys so far
        const float corr = __expf(M - mn);
        L *= corr;
#pragma unroll
        for (int e = 0; e < VPL; e++) A[e] *= corr;
#pragma unroll
        for (int u = 0; u < SB; u++) {
            const float c = __expf(mv[u] - mn);  // 0 for splits past the end
            L = fmaf(lv[u], c, L);
#pragma unroll
            for (int e = 0; e < VPL; e++) A[e] = fmaf(av[u][e], c, A[e]);
        }
        M = mn;
    }
    // the waves' results through step 3's LDS (free since the barriers above)
#pragma unroll
    for (int e = 0; e < VPL; e++) wacc[wave][gl][o0 - gl * Dh + e] = A[e];
    if ((o0 & (Dh - 1)) == 0) wm[wave][gl] = M, wl[wave][gl] = L;
    __syncthreads();
#pragma unroll
    for (int r = 0; r < PER; r++) {
        const int t = threadIdx.x + 256 * r;
        if (t < G * Dh) {
            const int g = t / Dh, d = t - g * Dh;
            float Mt = wm[0][g];
#pragma unroll
            for (int w = 1; w < 4; w++) Mt = fmaxf(Mt, wm[w][g]);
            float Lt = 0.0f, At = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const float c = wm[w][g] == -__builtin_inff() ? 0.0f : __expf(wm[w][g] - Mt);
                Lt = fmaf(wl[w][g], c, Lt);
                At = fmaf(wacc[w][g][d], c, At);
            }
            st_act(a.out, (int64_t)hk * G * Dh + t, marked ? __builtin_nanf("") : At / Lt, a.out_dt);
        }
    }
    if (threadIdx.x == 0) {
        __hip_atomic_store(a.sync + hk, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // every block of the XCD has arrived and every attention block's wait saw
    // every flag set: the flags start the next call at zero (after a wait that
    // gave up, a flag may still be set later, so they stay for the host's reset)
    if (FUSED && !marked)
        for (int i = threadIdx.x; i < a.nflags; i += 256) a.flags[i] = 0;
}

template <int G, int U, bool KF16>
__global__ __launch_bounds__(256) void attn_decode_kernel(AttnArgs a) {
    // 1-D grid with `sync`: block b = 8 t + x runs on XCD x and takes kv head
    // x + 8 (t / nsplit), split t % nsplit
    const int t8 = blockIdx.x >> 3;
    const int split = a.sync ? t8 % a.nsplit : blockIdx.x;
    const int hk = a.sync ? (blockIdx.x & 7) + 8 * (t8 / a.nsplit) : blockIdx.y;
    attn_body<G, U, false, KF16>(a, split, hk, [] { return false; });
}

// ---- the q/k/v product and the attention of one token in one launch ----------------
// Block b = 8 t + x runs on XCD x (workgroups are dealt round-robin) and owns kv
// head x (8 kv heads): first its share of the q/k/v rows of that head (the G
// query heads, the key head and the value head: (G + 2) x 128 rows of the
// stacked matrix, 8 rows per block pass, the decode GEMV tile <32,1,4,4> with
// the prepared-norm prologue, so the rows are bit for bit those of the plain
// product), stored (bf16 or f32); then it sets its own arrival flag. Blocks
// t < nsplit then run split t of the head's attention (attn_body): their K/V
// rows are requested at once, and the q/k/v rows are read device-coherently
// once one wave has seen every flag of the XCD set; the splits merge in the
// launch, whose last block clears the flags for the next call.
// (One arrival counter per XCD, 96 atomics on one L2 line, took 3-11 us to be
// seen by the pollers on MI355X; per-block flags, about 1 us.) Every block of the grid is resident at once
// (the launcher sizes the grid to the occupancy), so the wait ends. Its bound
// (`spin` polls) is a safety net that fails loudly: a wait that gives up marks
// its XCD, the head's output is NaN, the flags are not cleared, and `status`
// (host memory) is set for the library to report at the next synchronisation,
// where it resets the flags and markers. A marker left by an earlier call
// makes this call's heads on that XCD NaN as well.
struct QkvRows {
    uint32_t qbase, kbase, vbase, g128, nblk, past;
    __device__ uint32_t base(uint32_t blk) const {
        if (blk >= nblk) return past;
        const uint32_t i = blk * 8;
        return i < g128 ? qbase + i : (i < g128 + 128 ? kbase + (i - g128) : vbase + (i - g128 - 128));
    }
};

struct QkvAttnArgs {
    AttnArgs a;                 // a.qkv: the product's output (bf16 or f32); a.flags: set below per XCD
    int* flags;                 // per XCD kAttnMaxBlocksPerXcd arrival flags
    const uint32_t* w;          // stacked q/k/v rows [(Hq + 2 Hk) * 128, K / 8]
    const uint16_t* s;
    const uint16_t* b;
    const uint16_t* x;          // bf16 prepared norm input [K]
    float* stats;               // its sum-of-squares partials (kNormSlots)
    float norm_eps;
    int gs_log2;
    int bpx;                    // blocks per XCD
    uint32_t spin;              // polls of the flags before a wait gives up
    int* markers;               // per XCD give-up markers (device)
    int* status;                // set to 1 when a wait gives up (host memory the library reads)
};

template <int G, int U, bool KF16>
__global__ __launch_bounds__(256) void qkv_attn_kernel(QkvAttnArgs f) {
    const int x = blockIdx.x & 7, t = blockIdx.x >> 3;
    int* flags = f.flags + kAttnMaxBlocksPerXcd * x;
    AttnArgs a = f.a;
    a.flags = flags;
    a.marker = f.markers + x;
    const int Hq = a.Hk * G;
    const uint32_t rows = (uint32_t)(Hq + 2 * a.Hk) * 128;
    const QkvRows map{(uint32_t)(x * G * 128), (uint32_t)((Hq + x) * 128), (uint32_t)((Hq + a.Hk + x) * 128),
                      (uint32_t)(G * 128), (uint32_t)((G + 2) * 16), rows};
    qmvt::QmvFusion fu;
    fu.eps = f.norm_eps;
    fu.stats = f.stats;
    qmvt::qmv_tile<32, 1, 4, 4, false, qmvt::PRO_NORMED, qmvt::EPI_STORE, 4, false>(
        f.w, f.s, f.b, f.x, const_cast<void*>(a.qkv), a.qkv_dt, rows, f.gs_log2, fu, (uint32_t)t, (uint32_t)f.bpx,
        map.nblk, map);
    // the block's rows are in the L2 before its flag is
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_store(flags + t, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (t >= a.nsplit) return;
    attn_body<G, U, true, KF16>(a, t, x, [&]() -> bool {
        __shared__ int bad;
        // wave 0 reads all the XCD's flags per round (device-scope atomic loads:
        // they miss the L1, and the compiler keeps them in the loop)
        if (threadIdx.x < 64) {
            const int l = threadIdx.x;
            // a marker an earlier call left (not yet reset by the host)
            const int stale = __hip_atomic_load(a.marker, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            bool seen = false;
            for (uint32_t n = 0; n < f.spin; n++) {
                const int f0 = l < f.bpx ? __hip_atomic_load(flags + l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 1;
                const int f1 =
                    l + 64 < f.bpx ? __hip_atomic_load(flags + l + 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 1;
                if (__all(f0 == 1 && f1 == 1)) {
                    seen = true;
                    break;
                }
            }
            if (l == 0) {
                bad = !seen || stale != 0;
                if (!seen) {
                    // the marker reaches this XCD's L2 before the block's arrival
                    // (the partial stores' wait covers it); the status word is
                    // read by the host after the stream's work is done
                    __hip_atomic_store(a.marker, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(f.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                }
            }
        }
        __syncthreads();
        return bad != 0;
    });
}

// Workgroup -> XCD placement: out[b] = the XCD (XCC id) block b runs on, b the
// block's index in dispatch order (x fastest, then y, then z).
__global__ __launch_bounds__(64) void xcc_probe_kernel(int* out) {
    unsigned x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
    const unsigned b = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
    if (threadIdx.x == 0) out[b] = (int)(x & 0xFu);
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

// ---- Argmax: first index of the maximum; blocks take chunks, one block merges ----
constexpr int kArgmaxChunks = 128;

__device__ __forceinline__ void better(float& bv, int64_t& bi, float v, int64_t i) {
    if (v > bv || (v == bv && i < bi)) bv = v, bi = i;
}

// Block (chunk c, row r): the best (value, index) of chunk c of row r, with the
// loads of each thread issued together.
__global__ __launch_bounds__(256) void argmax_partial_kernel(const void* __restrict__ x, int x_dt, int64_t n,
                                                             float* __restrict__ pv, int64_t* __restrict__ pi) {
    __shared__ float sv[4];
    __shared__ int64_t si[4];
    const int64_t r = blockIdx.y;
    const int64_t chunk = (n + kArgmaxChunks - 1) / kArgmaxChunks;
    const int64_t lo = blockIdx.x * chunk, hi = min(n, lo + chunk);
    float best = -__builtin_inff();
    int64_t idx = n;  // "none": loses every tie
    constexpr int U = 8;
    for (int64_t i0 = lo + threadIdx.x; i0 < hi; i0 += 256 * U) {
        float v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int64_t i = i0 + (int64_t)u * 256;
            v[u] = i < hi ? ld_act(x, r * n + i, x_dt) : -__builtin_inff();
        }
#pragma unroll
        for (int u = 0; u < U; u++)
            if (v[u] > best) best = v[u], idx = i0 + (int64_t)u * 256;  // ascending i per thread
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) better(best, idx, __shfl_xor(best, o, 64), __shfl_xor(idx, o, 64));
    if ((threadIdx.x & 63) == 0) sv[threadIdx.x >> 6] = best, si[threadIdx.x >> 6] = idx;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < 4; k++) better(best, idx, sv[k], si[k]);
        pv[r * kArgmaxChunks + blockIdx.x] = best;
        pi[r * kArgmaxChunks + blockIdx.x] = idx;
    }
}

__global__ __launch_bounds__(128) void argmax_final_kernel(const float* __restrict__ pv, const int64_t* __restrict__ pi,
                                                           int64_t n, int32_t* __restrict__ out) {
    const int64_t r = blockIdx.x;
    float best = pv[r * kArgmaxChunks + threadIdx.x];
    int64_t idx = pi[r * kArgmaxChunks + threadIdx.x];
    __shared__ float sv[2];
    __shared__ int64_t si[2];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) better(best, idx, __shfl_xor(best, o, 64), __shfl_xor(idx, o, 64));
    if ((threadIdx.x & 63) == 0) sv[threadIdx.x >> 6] = best, si[threadIdx.x >> 6] = idx;
    __syncthreads();
    if (threadIdx.x == 0) {  // holds wave 0's result
        better(best, idx, sv[1], si[1]);
        out[r] = idx < n ? (int32_t)idx : 0;
    }
}

// One launch: argmax_partial_kernel's blocks, then the last block of row r to
// arrive (counted at sync[r], across all XCDs: agent-scope fences around the
// count) reduces the row's candidates as argmax_final_kernel does and resets
// the counter. The result does not depend on arrival order (better() is a
// total order on (value, index)).
__global__ __launch_bounds__(256) void argmax_one_kernel(const void* __restrict__ x, int x_dt, int64_t n,
                                                         float* __restrict__ pv, int64_t* __restrict__ pi,
                                                         int* __restrict__ sync, int32_t* __restrict__ out) {
    __shared__ float sv[4];
    __shared__ int64_t si[4];
    __shared__ int last;
    const int64_t r = blockIdx.y;
    const int64_t chunk = (n + kArgmaxChunks - 1) / kArgmaxChunks;
    const int64_t lo = blockIdx.x * chunk, hi = min(n, lo + chunk);
    float best = -__builtin_inff();
    int64_t idx = n;
    constexpr int U = 8;
    for (int64_t i0 = lo + threadIdx.x; i0 < hi; i0 += 256 * U) {
        float v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int64_t i = i0 + (int64_t)u * 256;
            v[u] = i < hi ? ld_act(x, r * n + i, x_dt) : -__builtin_inff();
        }
#pragma unroll
        for (int u = 0; u < U; u++)
            if (v[u] > best) best = v[u], idx = i0 + (int64_t)u * 256;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) better(best, idx, __shfl_xor(best, o, 64), __shfl_xor(idx, o, 64));
    if ((threadIdx.x & 63) == 0) sv[threadIdx.x >> 6] = best, si[threadIdx.x >> 6] = idx;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < 4; k++) better(best, idx, sv[k], si[k]);
        pv[r * kArgmaxChunks + blockIdx.x] = best;
        pi[r * kArgmaxChunks + blockIdx.x] = idx;
        __threadfence();  // the candidate is visible device-wide before the arrival
        last = atomicAdd(sync + r, 1) == kArgmaxChunks - 1;
    }
    __syncthreads();
    if (!last) return;
    __threadfence();  // and every other block's candidate is seen here
    if (threadIdx.x < kArgmaxChunks) {
        best = pv[r * kArgmaxChunks + threadIdx.x];
        idx = pi[r * kArgmaxChunks + threadIdx.x];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) better(best, idx, __shfl_xor(best, o, 64), __shfl_xor(idx, o, 64));
        if ((threadIdx.x & 63) == 0) sv[threadIdx.x >> 6] = best, si[threadIdx.x >> 6] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        better(best, idx, sv[1], si[1]);
        out[r] = idx < n ? (int32_t)idx : 0;
        sync[r] = 0;
    }
}

// ---- row gather and KV append ------------------------------------------------------
// ---- strided copy with conversion (Slice / Transpose / Concat / Cast / contiguous) --
// dst = src over `shape`, each side addressed through its own element strides,
// converted between F32/F16/BF16; I32/U32/U8 copy only to their own type.
struct NdDesc {
    int nd;
    int64_t shape[kMaxCopyDims];
    int64_t stride[kMaxCopyDims];   // src
    int64_t dstride[kMaxCopyDims];  // dst
};

__device__ __forceinline__ int elem_bytes(int dt) { return dt == JH_F32 || dt == JH_I32 || dt == JH_U32 ? 4 : dt == JH_U8 ? 1 : 2; }

__global__ __launch_bounds__(256) void copy_strided_kernel(const void* __restrict__ src, int sdt,
                                                           void* __restrict__ dst, int ddt, int64_t n, NdDesc d) {
    const bool raw = sdt == ddt;
    const int eb = elem_bytes(sdt);
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        int64_t rem = i, off = 0, doff = 0;
        for (int a = d.nd - 1; a >= 0; a--) {
            const int64_t c = rem % d.shape[a];
            rem /= d.shape[a];
            off += c * d.stride[a];
            doff += c * d.dstride[a];
        }
        if (raw) {
            if (eb == 4) static_cast<uint32_t*>(dst)[doff] = static_cast<const uint32_t*>(src)[off];
            else if (eb == 2) static_cast<uint16_t*>(dst)[doff] = static_cast<const uint16_t*>(src)[off];
            else static_cast<uint8_t*>(dst)[doff] = static_cast<const uint8_t*>(src)[off];
            continue;
        }
        const float v = ld_act(src, off, sdt);
        if (ddt == JH_F16)
            static_cast<uint16_t*>(dst)[doff] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
        else
            st_act(dst, doff, v, ddt);
    }
}

__global__ __launch_bounds__(256) void take_rows_kernel(const uint8_t* __restrict__ table, int64_t row_bytes,
                                                        int64_t n_rows, const int32_t* __restrict__ ids,
                                                        uint8_t* __restrict__ out) {
    const int64_t k = blockIdx.x;
    const int32_t id = ids[k];
    const bool ok = id >= 0 && id < n_rows;
    for (int64_t i = threadIdx.x; i < row_bytes; i += 256)
        out[k * row_bytes + i] = ok ? table[(int64_t)id * row_bytes + i] : (uint8_t)0;
}

// Row copies of a scatter: block (x, y) copies bytes [x * kScatterChunk, ...)
// of update row l.src[y] into out row l.dst[y], in `vec`-byte words (16 when
// the row length and both bases allow it, else 4, else 1).
__global__ __launch_bounds__(256) void scatter_rows_kernel(ScatterList l, const uint8_t* __restrict__ upd,
                                                           uint8_t* __restrict__ out, int64_t row_bytes, int vec) {
    const int e = blockIdx.y;
    const uint8_t* s = upd + (int64_t)l.src[e] * row_bytes;
    uint8_t* d = out + (int64_t)l.dst[e] * row_bytes;
    const int64_t lo = (int64_t)blockIdx.x * kScatterChunk;
    const int64_t hi = min(row_bytes, lo + (int64_t)kScatterChunk);
    if (vec == 16) {
        for (int64_t i = lo + 16 * threadIdx.x; i < hi; i += 16 * 256)
            *reinterpret_cast<uint4*>(d + i) = *reinterpret_cast<const uint4*>(s + i);
    } else if (vec == 4) {
        for (int64_t i = lo + 4 * threadIdx.x; i < hi; i += 4 * 256)
            *reinterpret_cast<uint32_t*>(d + i) = *reinterpret_cast<const uint32_t*>(s + i);
    } else {
        for (int64_t i = lo + threadIdx.x; i < hi; i += 256) d[i] = s[i];
    }
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
    if (rows > 0x7fffffff / 4) return Status::fail(JH_ERR_UNSUPPORTED, "rms_norm: too many rows");
    const dim3 wg((unsigned)((rows + 3) / 4)), bg((unsigned)rows);
    auto wave = [&](auto k) { hipLaunchKernelGGL(k, wg, dim3(256), 0, st, x, x_dt, w, w_dt, eps, out, out_dt, rows, d); };
    auto block = [&](auto k) { hipLaunchKernelGGL(k, bg, dim3(256), 0, st, x, x_dt, w, w_dt, eps, out, out_dt, d); };
    if (d <= 128) wave(rms_norm_wave_kernel<2>);
    else if (d <= 256) wave(rms_norm_wave_kernel<4>);
    else if (d <= 1024) wave(rms_norm_wave_kernel<16>);
    else if (d <= 4096) block(rms_norm_block_kernel<16>);
    else if (d <= 8192) block(rms_norm_block_kernel<32>);
    else if (d <= 16384) block(rms_norm_block_kernel<64>);
    else block(rms_norm_long_kernel);
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
    return Lq == 1 && Dh == kDecodeDh && (kv_dt == JH_BF16 || kv_dt == JH_F16) && (G == 1 || G == 2 || G == 4 || G == 8) &&
           (q_dt == JH_BF16 || q_dt == JH_F32);
}

int64_t sdpa_splits(int64_t B, int64_t Hk, int64_t Lk, int num_cus) {
    // at least two blocks per CU and at most 64 keys per block, but no fewer
    // than 16 keys per block (one per key slot)
    int64_t n = (2 * (int64_t)num_cus + B * Hk - 1) / (B * Hk);
    n = std::max<int64_t>(n, (Lk + 63) / 64);
    n = std::min<int64_t>(n, (Lk + 15) / 16);
    n = std::min<int64_t>(n, kMaxSplits);
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
        const bool f16 = kv_dt == JH_F16;
        if (G == 1) f16 ? go(sdpa_decode_split_kernel<1, true>) : go(sdpa_decode_split_kernel<1, false>);
        else if (G == 2) f16 ? go(sdpa_decode_split_kernel<2, true>) : go(sdpa_decode_split_kernel<2, false>);
        else if (G == 4) f16 ? go(sdpa_decode_split_kernel<4, true>) : go(sdpa_decode_split_kernel<4, false>);
        else f16 ? go(sdpa_decode_split_kernel<8, true>) : go(sdpa_decode_split_kernel<8, false>);
        hipLaunchKernelGGL(sdpa_decode_merge_kernel, dim3((unsigned)(B * Hq)), dim3(kDecodeDh * merge_groups(nsplit)), 0, st,
                           part, (int)Hk, G,
                           (int)nsplit, out, out_dt);
        return Status::ok();
    }
    if (Dh > 256) return Status::fail(JH_ERR_UNSUPPORTED, "sdpa: head_dim above 256");
    hipLaunchKernelGGL(sdpa_rows_kernel, dim3((unsigned)(B * Hq * Lq)), dim3(256), 0, st, q, q_dt, k, v, kv_dt, out,
                       out_dt, (int)Hq, (int)Hk, (int)Lq, (int)Lk, (int)kcap, (int)Dh, scale, causal ? 1 : 0);
    return Status::ok();
}

Status launch_qk_norm_rope_append(const void* qkv, int qkv_dt, int Hq, int Hk, const void* qn_w, const void* kn_w,
                                  int w_dt, float eps, float base, float scale, int64_t pos, void* kc, void* vc,
                                  int c_dt, int64_t cap, void* q_out, int q_dt, hipStream_t st) {
    const int heads = Hq + 2 * Hk;
    hipLaunchKernelGGL(qk_norm_rope_append_kernel, dim3((unsigned)((heads + 3) / 4)), dim3(256), 0, st, qkv, qkv_dt, Hq,
                       Hk, qn_w, kn_w, w_dt, eps, base, scale, pos, kc, vc, c_dt, cap, q_out, q_dt);
    return Status::ok();
}

// The split of the `pos` cache rows over blocks: one load batch per slot where
// possible (all of a block's K/V rows requested at once: a second batch waits a
// whole memory latency), 4 keys per slot while that keeps the grid within about
// 2 blocks per CU over the kv heads, else 8 (two such blocks fit a CU), and
// several batches per block beyond that. The new key joins the last split, so
// the grid stays within the target (the two-blocks-per-CU occupancy of the
// 8-key kernel).
struct AttnSplit {
    int u;          // keys per slot per batch
    int64_t kps;    // cache rows per split
    int64_t nsplit;
    bool owner_alone;
};

// With the in-launch merge the last block reads every split's partials, so
// long caches take one block per CU instead of two (the attention launch alone
// measured the same for 128 to 1024 blocks at 8192 keys).
AttnSplit attn_split(int64_t Hk, int64_t pos, int num_cus, bool in_launch) {
    const int64_t target = std::max<int64_t>(1, (in_launch ? 1 : 2) * (int64_t)num_cus / Hk);
    AttnSplit sp;
    sp.u = pos <= 64 * target ? 4 : 8;
    const int64_t batch = 16 * sp.u;
    sp.kps = batch * std::max<int64_t>(1, (pos + batch * target - 1) / (batch * target));
    const int64_t cache_splits = (pos + sp.kps - 1) / sp.kps;
    // the new key's own block keeps its q/k/v work off the longest block's path,
    // when the grid has room for it
    sp.owner_alone = cache_splits + 1 <= target || cache_splits == 0;
    sp.nsplit = sp.owner_alone ? cache_splits + 1 : cache_splits;
    return sp;
}

size_t attn_decode_workspace_bytes(int64_t Hq, int64_t Hk, int64_t pos, int num_cus) {
    // the larger of the two plans' needs
    AttnSplit sp = attn_split(Hk, pos, num_cus, false);
    const AttnSplit sp1 = attn_split(Hk, pos, num_cus, true);
    if (sp1.nsplit > sp.nsplit) sp = sp1;
    if (sp.nsplit <= 1) return 0;
    // the larger of the two layouts (records padded to whole lines for the
    // in-launch merge)
    const int64_t G = Hq / Hk;
    const int64_t rec = std::max<int64_t>(G * (kDecodeDh + 2), (G * (kDecodeDh + 2) + 31) / 32 * 32);
    return (size_t)(Hk * sp.nsplit * rec) * sizeof(float);
}

bool attn_merge_in_launch(int64_t Hk, const int* sync) { return sync != nullptr && Hk % 8 == 0 && Hk <= kAttnFlagSlot; }

namespace {
int log2_exact(int v) {
    int l = 0;
    while ((1 << l) < v) l++;
    return ((1 << l) == v) ? l : -1;
}
}  // namespace

// The fused launch takes 8 kv heads (one per XCD) of head_dim 128, G = 1, 2, 4
// or 8, and the q/k/v matrix the <32,1,4,4> decode tile takes: K = 4096, 4-bit
// codes in groups of 64 with bf16 scales, (Hq + 2 Hk) x 128 rows.
bool qkv_attn_ok(const QuantMatrix& m, int64_t Hq, int64_t Hk, const int* sync, int num_cus) {
    const int64_t G = Hk > 0 ? Hq / Hk : 0;
    return sync != nullptr && Hk == 8 && G * Hk == Hq && (G == 1 || G == 2 || G == 4 || G == 8) && m.bits == 4 &&
           m.group_size == 64 && m.in == 4096 && m.sb_dtype == JH_BF16 && m.rows == (Hq + 2 * Hk) * kDecodeDh &&
           num_cus % 8 == 0 && num_cus >= 64;
}

Status launch_attn_decode(const void* qkv, int qkv_dt, int Hq, int Hk, const void* qn_w, const void* kn_w, int w_dt,
                          float eps, float base, float rscale, const float* rope_cs, int64_t pos, void* kc,
                          void* vc, int c_dt, int64_t cap, float scale, void* out, int out_dt, void* workspace,
                          int num_cus, hipStream_t st, int* sync) {
    const int G = Hq / Hk;
    const bool sync_ok = attn_merge_in_launch(Hk, sync);
    const AttnSplit sp = attn_split(Hk, pos, num_cus, sync_ok);
    const int64_t kps = sp.kps, nsplit = sp.nsplit;
    if (nsplit > kMaxSplits || kps > 0x7fffffff) return Status::fail(JH_ERR_UNSUPPORTED, "attention: cache too long");
    // cache rows are addressed with 32-bit byte offsets within a head
    if (cap > ((int64_t)1 << 23) - 1024) return Status::fail(JH_ERR_UNSUPPORTED, "attention: capacity above 8M tokens");
    const bool in_launch = nsplit > 1 && sync_ok;
    AttnArgs a{qkv, qkv_dt, qn_w, kn_w, w_dt, eps, base, rscale, scale, rope_cs, pos,
               static_cast<uint16_t*>(kc), static_cast<uint16_t*>(vc), cap, Hk, (int)nsplit, (int)kps,
               sp.owner_alone ? 1 : 0, static_cast<float*>(workspace), out, out_dt, in_launch ? sync : nullptr};
    const dim3 grid = in_launch ? dim3((unsigned)(nsplit * Hk)) : dim3((unsigned)nsplit, (unsigned)Hk);
    const bool u8 = sp.u == 8;
    auto go = [&](auto k4, auto k8) {
        if (u8)
            hipLaunchKernelGGL(k8, grid, dim3(256), 0, st, a);
        else
            hipLaunchKernelGGL(k4, grid, dim3(256), 0, st, a);
    };
    auto go_dt = [&](auto b4, auto b8, auto h4, auto h8) { c_dt == JH_F16 ? go(h4, h8) : go(b4, b8); };
    if (G == 1)
        go_dt(attn_decode_kernel<1, 4, false>, attn_decode_kernel<1, 8, false>, attn_decode_kernel<1, 4, true>,
              attn_decode_kernel<1, 8, true>);
    else if (G == 2)
        go_dt(attn_decode_kernel<2, 4, false>, attn_decode_kernel<2, 8, false>, attn_decode_kernel<2, 4, true>,
              attn_decode_kernel<2, 8, true>);
    else if (G == 4)
        go_dt(attn_decode_kernel<4, 4, false>, attn_decode_kernel<4, 8, false>, attn_decode_kernel<4, 4, true>,
              attn_decode_kernel<4, 8, true>);
    else if (G == 8)
        go_dt(attn_decode_kernel<8, 4, false>, attn_decode_kernel<8, 8, false>, attn_decode_kernel<8, 4, true>,
              attn_decode_kernel<8, 8, true>);
    else return Status::fail(JH_ERR_UNSUPPORTED, "attention: n_heads / n_kv_heads must be 1, 2, 4 or 8");
    if (nsplit > 1 && !in_launch)
        hipLaunchKernelGGL(sdpa_decode_merge_kernel, dim3((unsigned)Hq), dim3(kDecodeDh * merge_groups(nsplit)), 0, st,
                           static_cast<const float*>(workspace), Hk, G, (int)nsplit, out, out_dt);
    return Status::ok();
}

Status launch_qkv_attn(const QuantMatrix& m, const uint16_t* x, float* stats, float norm_eps, void* qkv, int qkv_dt,
                       int Hq, int Hk, const void* qn_w, const void* kn_w, int w_dt, float eps, float base, float rscale,
                       const float* rope_cs, int64_t pos, void* kc, void* vc, int c_dt, int64_t cap, float scale,
                       void* out, int out_dt, void* workspace, int num_cus, hipStream_t st, int* sync,
                       uint32_t spin, int* status) {
    const int G = Hk > 0 ? Hq / Hk : 0;
    if (!qkv_attn_ok(m, Hq, Hk, sync, num_cus)) return Status::fail(JH_ERR_UNSUPPORTED, "qkv_attn: outside the fused launch");
    if (cap > ((int64_t)1 << 23) - 1024) return Status::fail(JH_ERR_UNSUPPORTED, "attention: capacity above 8M tokens");
    const AttnSplit sp = attn_split(Hk, pos, num_cus, true);
    const bool u8 = sp.u == 8;
    // blocks per XCD: one per 8-row pass of the head's q/k/v rows, at most what
    // is resident at once (the attention blocks wait for all of them)
    auto go = [&](auto k4, auto k8) -> Status {
        auto kern = u8 ? k8 : k4;
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, 256, 0) != hipSuccess || per_cu < 1) {
            (void)hipGetLastError();
            return Status::fail(JH_ERR_UNSUPPORTED, "qkv_attn: occupancy unknown");
        }
        // two blocks per CU at most: against three (the occupancy of the 4-key
        // kernel) the whole decode step measured 36-44 us per token faster at 512
        // keys and 20 us at 8192 on MI355X (the product phase's last blocks
        // finished ~2 us later with three); one block per CU was slower than both
        per_cu = std::min(per_cu, 2);
        const int bpx = std::min({(G + 2) * 16, per_cu * (num_cus / 8), kAttnMaxBlocksPerXcd});
        if (bpx < sp.nsplit) return Status::fail(JH_ERR_UNSUPPORTED, "qkv_attn: more splits than resident blocks");
        QkvAttnArgs f{};
        f.a = AttnArgs{qkv, qkv_dt, qn_w, kn_w, w_dt, eps, base, rscale, scale, rope_cs, pos,
                       static_cast<uint16_t*>(kc), static_cast<uint16_t*>(vc), cap, Hk, (int)sp.nsplit, (int)sp.kps,
                       sp.owner_alone ? 1 : 0, static_cast<float*>(workspace), out, out_dt,
                       sp.nsplit > 1 ? sync : nullptr, nullptr, bpx};
        f.flags = sync + kAttnFlagSlot;
        f.w = m.w;
        f.s = static_cast<const uint16_t*>(m.scales);
        f.b = static_cast<const uint16_t*>(m.biases);
        f.x = x;
        f.stats = stats;
        f.norm_eps = norm_eps;
        f.gs_log2 = log2_exact(m.group_size);
        f.bpx = bpx;
        f.spin = spin;
        f.markers = sync + kAttnMarkerSlot;
        f.status = status;
        hipLaunchKernelGGL(kern, dim3((unsigned)(8 * bpx)), dim3(256), 0, st, f);
        return Status::ok();
    };
    const bool f16 = c_dt == JH_F16;
    if (G == 1)
        return f16 ? go(qkv_attn_kernel<1, 4, true>, qkv_attn_kernel<1, 8, true>)
                   : go(qkv_attn_kernel<1, 4, false>, qkv_attn_kernel<1, 8, false>);
    if (G == 2)
        return f16 ? go(qkv_attn_kernel<2, 4, true>, qkv_attn_kernel<2, 8, true>)
                   : go(qkv_attn_kernel<2, 4, false>, qkv_attn_kernel<2, 8, false>);
    if (G == 4)
        return f16 ? go(qkv_attn_kernel<4, 4, true>, qkv_attn_kernel<4, 8, true>)
                   : go(qkv_attn_kernel<4, 4, false>, qkv_attn_kernel<4, 8, false>);
    return f16 ? go(qkv_attn_kernel<8, 4, true>, qkv_attn_kernel<8, 8, true>)
               : go(qkv_attn_kernel<8, 4, false>, qkv_attn_kernel<8, 8, false>);
}

int probe_xcd_round_robin(int* buf, hipStream_t st) {
    // a 1-D grid (the attention launches) and a 3-D one (the split-K product:
    // x by columns, y by rows, z by K split)
    constexpr int kBlocks = 64;
    hipLaunchKernelGGL(xcc_probe_kernel, dim3(kBlocks), dim3(64), 0, st, buf);
    hipLaunchKernelGGL(xcc_probe_kernel, dim3(4, 2, 8), dim3(64), 0, st, buf + kBlocks);
    int h[2 * kBlocks];
    if (hipMemcpyAsync(h, buf, sizeof h, hipMemcpyDeviceToHost, st) != hipSuccess || hipStreamSynchronize(st) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    for (int b = 0; b < 2 * kBlocks; b++)
        if (h[b] != b % 8) return 0;
    return 8;
}

Status launch_norm_prepare(const void* x, int x_dt, int64_t d, const void* w, int w_dt, uint16_t* out, float* stats,
                           hipStream_t st) {
    const int64_t blocks = (d + 256 * kPrepPer - 1) / (256 * kPrepPer);
    if (blocks > kNormSlots) return Status::fail(JH_ERR_UNSUPPORTED, "norm_prepare: row too long");
    hipLaunchKernelGGL(norm_prepare_kernel, dim3((unsigned)blocks), dim3(256), 0, st, x, x_dt, d, w, w_dt, out, stats);
    return Status::ok();
}

Status launch_embed_norm(const int32_t* ids, const QuantMatrix& m, const void* w, int w_dt, float* h, uint16_t* out,
                         float* stats, int rope_dims, float base, float scale, int64_t pos, float* cs, hipStream_t st) {
    const int64_t nb = (m.in + 256 * kPrepPer - 1) / (256 * kPrepPer);
    if (nb > kNormSlots) return Status::fail(JH_ERR_UNSUPPORTED, "embed_norm: row too long");
    const dim3 grid((unsigned)(nb + (cs ? 1 : 0)));
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, dim3(256), 0, st, ids, m.w, m.scales, m.biases, m.sb_dtype, m.rows, m.in,
                           m.group_size, w, w_dt, h, out, stats, (int)nb, rope_dims, base, scale, pos, cs);
    };
    if (m.bits == 8) go(embed_norm_kernel<8>);
    else if (m.bits == 2) go(embed_norm_kernel<2>);
    else go(embed_norm_kernel<4>);
    return Status::ok();
}

Status launch_norm_apply(const uint16_t* u, int64_t d, const float* stats, float eps, uint16_t* out, hipStream_t st) {
    hipLaunchKernelGGL(norm_apply_kernel, dim3(1), dim3(256), 0, st, u, d, stats, eps, out);
    return Status::ok();
}

Status launch_rope_table(int dims, float base, float scale, int64_t pos, const float* freqs, float* out,
                         hipStream_t st) {
    hipLaunchKernelGGL(rope_table_kernel, dim3(1), dim3(64), 0, st, dims, base, scale, pos, freqs, out);
    return Status::ok();
}

Status launch_elementwise(int op, const void* a, int a_dt, const void* b, int b_dt, void* out, int out_dt, int64_t n,
                          hipStream_t st) {
    if (n == 0) return Status::ok();
    hipLaunchKernelGGL(elementwise_kernel, dim3(grid_for(n, 256, 16384)), dim3(256), 0, st, op, a, a_dt, b, b_dt, out,
                       out_dt, n);
    return Status::ok();
}

size_t argmax_workspace_bytes(int64_t rows) { return (size_t)rows * kArgmaxChunks * (sizeof(float) + sizeof(int64_t)); }

Status launch_argmax(const void* x, int x_dt, int64_t rows, int64_t n, int32_t* out, void* workspace, int* sync,
                     hipStream_t st) {
    if (rows == 0) return Status::ok();
    if (rows > 65535) return Status::fail(JH_ERR_UNSUPPORTED, "argmax: more than 65535 rows");
    int64_t* pi = static_cast<int64_t*>(workspace);
    float* pv = reinterpret_cast<float*>(pi + rows * kArgmaxChunks);
    if (sync && rows <= kArgmaxSyncRows) {
        hipLaunchKernelGGL(argmax_one_kernel, dim3(kArgmaxChunks, (unsigned)rows), dim3(256), 0, st, x, x_dt, n, pv,
                           pi, sync + kArgmaxSyncSlot, out);
        return Status::ok();
    }
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(kArgmaxChunks, (unsigned)rows), dim3(256), 0, st, x, x_dt, n, pv, pi);
    hipLaunchKernelGGL(argmax_final_kernel, dim3((unsigned)rows), dim3(kArgmaxChunks), 0, st, pv, pi, n, out);
    return Status::ok();
}

Status launch_copy_strided(const void* src, int sdt, int nd, const int64_t* shape, const int64_t* strides, void* dst,
                           int ddt, const int64_t* dst_strides, hipStream_t st) {
    NdDesc d{};
    d.nd = nd;
    int64_t n = 1;
    for (int a = nd - 1; a >= 0; a--) {
        d.shape[a] = shape[a];
        d.stride[a] = strides[a];
        d.dstride[a] = dst_strides ? dst_strides[a] : n;  // contiguous by default
        n *= shape[a];
    }
    if (n == 0) return Status::ok();
    hipLaunchKernelGGL(copy_strided_kernel, dim3(grid_for(n, 256, 16384)), dim3(256), 0, st, src, sdt, dst, ddt, n, d);
    return Status::ok();
}

Status launch_scatter_rows(const ScatterList& l, const void* updates, void* out, int64_t row_bytes,
                           hipStream_t st) {
    if (l.n <= 0 || row_bytes <= 0) return Status::ok();
    const int64_t chunks = (row_bytes + kScatterChunk - 1) / kScatterChunk;
    if (chunks > 0x7fffffff) return Status::fail(JH_ERR_UNSUPPORTED, "scatter_rows: rows too long");
    const auto aligned = [](const void* p, int a) { return reinterpret_cast<uintptr_t>(p) % a == 0; };
    const int vec = row_bytes % 16 == 0 && aligned(updates, 16) && aligned(out, 16) ? 16
                    : row_bytes % 4 == 0 && aligned(updates, 4) && aligned(out, 4)  ? 4
                                                                                      : 1;
    hipLaunchKernelGGL(scatter_rows_kernel, dim3((unsigned)chunks, (unsigned)l.n), dim3(256), 0, st, l,
                       static_cast<const uint8_t*>(updates), static_cast<uint8_t*>(out), row_bytes, vec);
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
