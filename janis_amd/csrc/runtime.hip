// C ABI of libjanis_hip.so (include/janis_hip.h): context, memory, argument
// checking and dispatch of the quantized-linear operators to their kernels.
//
// Dispatch mirrors the reference's QuantMatmul (cpu/cpu_misc.go:232-400):
// rows == 1 is the decode GEMV (qmv.hip), rows > 1 the prefill GEMM (qmm.hip);
// GatherQuantMatmul buckets by expert on the device (gather.hip).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "jh_common.hpp"

struct jh_ctx {
    int device = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    int num_cus = 256;
    int checks = 0;
    char name[256] = {0};
    std::string err;
    void* ws = nullptr;  // operator workspace, grown on demand
    size_t ws_bytes = 0;
    // Workspaces replaced by a larger one. They stay allocated until jh_destroy:
    // a HIP graph captured earlier holds their address in its launches, and
    // replaying it must not touch memory that was freed (or reused since).
    std::vector<void*> retired;
    unsigned long long* check_buf = nullptr;  // 2 counters of the value checks
    void* scratch = nullptr;  // this device's copy of `scratch` (jh_attention_decode_noalloc)
    // Arrival counters of the in-launch attention merge (jh::kAttnSyncSlots
    // ints, zero between calls), or nullptr when the GPU does not deal
    // workgroups to its XCDs round-robin: then the merge is a second launch.
    int* attn_sync = nullptr;
    // The stream operators are enqueued on keeps the round-robin placement the
    // in-launch merges rely on (false for a stream restricted to some CUs).
    bool stream_xcd_ok = true;
    // Set by a fused launch whose in-kernel wait gave up (host memory the kernel
    // writes); read after every synchronisation (jh_sync, jh_d2h).
    int* wait_status = nullptr;
    uint32_t wait_polls = jh::kDefaultWaitPolls;
};

namespace {

thread_local std::string g_create_error;

// Scratch memory of jh_attention_decode_noalloc: a fixed device array, so that
// entry point never allocates. Each GPU the library runs on holds its own copy
// until the process ends. Its device address is taken once per device, with
// that device current, by hipGetSymbolAddress (in jh_create); host code uses
// that address only -- the array's name in host code is a host-side stand-in.
constexpr size_t kScratchBytes = (size_t)4 << 20;
__device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// This device's address of `scratch` (device current on this thread), or nullptr.
void* scratch_address(int device) {
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
        g_scratch_ptr[device] = p;
    }
    return g_scratch_ptr[device];
}

int fail(jh_ctx* c, int code, const std::string& msg) {
    if (c) c->err = msg;
    return code;
}

int hip_fail(jh_ctx* c, hipError_t e, const char* what) {
    return fail(c, JH_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

#define JH_HIP(ctx, call)                                      \
    do {                                                       \
        hipError_t e_ = (call);                                \
        if (e_ != hipSuccess) return hip_fail((ctx), e_, #call); \
    } while (0)

// Makes ctx's device current on this thread (hipSetDevice is per thread).
int enter(jh_ctx* c) {
    if (!c) return JH_ERR_INVALID;
    c->err.clear();
    JH_HIP(c, hipSetDevice(c->device));
    return JH_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Grows the context's workspace to at least `need` bytes (power of two, >= 4 KiB).
// The old buffer is retired, not freed (graphs captured before may replay into
// it), so growth never waits for the stream. Growth while the context's stream
// is being captured is refused: an allocation is not a stream operation, and a
// graph must not depend on one made during its capture; one eager call of the
// same operator and size before the capture sizes the workspace.
int ensure_workspace(jh_ctx* c, size_t need, const char* op) {
    if (need <= c->ws_bytes) return JH_OK;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    JH_HIP(c, hipStreamIsCapturing(c->stream, &cs));
    if (cs != hipStreamCaptureStatusNone)
        return fail(c, JH_ERR_INVALID,
                    std::string(op) + ": needs a workspace of " + std::to_string(need) + " bytes while the stream is " +
                        "being captured (the context holds " + std::to_string(c->ws_bytes) +
                        "); make the same call once before the capture");
    if (need > ((size_t)1 << 62)) return fail(c, JH_ERR_OOM, std::string(op) + ": workspace size overflows");
    size_t cap = 4096;
    while (cap < need) cap *= 2;
    void* p = nullptr;
    const hipError_t e = hipMalloc(&p, cap);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(c, JH_ERR_OOM, std::string(op) + ": workspace allocation of " + std::to_string(cap) +
                                       " bytes failed (" + hipGetErrorString(e) + ")");
    }
    if (c->ws) c->retired.push_back(c->ws);
    c->ws = p;
    c->ws_bytes = cap;
    return JH_OK;
}

int check_quant(jh_ctx* c, const char* op, const uint32_t* w, const void* s, const void* b,
                int sb_dtype, int64_t rows, int64_t in, int group_size, int bits) {
    if (bits != 2 && bits != 4 && bits != 8)
        return fail(c, JH_ERR_UNSUPPORTED,
                    std::string(op) + ": bits must be 2, 4 or 8 (32/bits codes per word; bits=" +
                        std::to_string(bits) + ")");
    if (sb_dtype != JH_BF16 && sb_dtype != JH_F16 && sb_dtype != JH_F32)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": scales/biases must be bf16, f16 or f32");
    if (rows < 0 || in <= 0)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": bad shape");
    if (in % (32 / bits) != 0)
        return fail(c, JH_ERR_INVALID,
                    std::string(op) + ": in_features must be a multiple of " + std::to_string(32 / bits) +
                        " (codes per word)");
    if (group_size <= 0 || in % group_size != 0)
        return fail(c, JH_ERR_INVALID,
                    std::string(op) + ": group_size " + std::to_string(group_size) +
                        " does not divide in_features " + std::to_string(in));
    if (rows > 0 && (!w || !s || !b))
        return fail(c, JH_ERR_INVALID, std::string(op) + ": null weight pointer");
    if (!aligned16(w))
        return fail(c, JH_ERR_INVALID, std::string(op) + ": weight pointer not 16-byte aligned");
    return JH_OK;
}

// The in-launch merge counters, when the context's stream keeps the
// round-robin workgroup placement (else nullptr: merges are launches of their own).
int* xcd_sync(const jh_ctx* c) { return c->stream_xcd_ok ? c->attn_sync : nullptr; }

// What a split-K prefill product needs to add its partial tiles inside its own
// launch (counters nullptr: a summing launch follows instead).
jh::InLaunchSync qmm_sync(const jh_ctx* c) {
    int* sync = xcd_sync(c);
    if (!sync || !c->wait_status) return {};
    return {sync + jh::kQmmSyncSlot, c->wait_polls, c->wait_status};
}

// After the stream's work is done: a fused launch whose in-kernel wait gave up
// left its status word set. Its heads' outputs are NaN; the flags and markers it
// left are reset here (the stream is idle) and the failure is reported.
int check_wait_status(jh_ctx* c, const char* op) {
    if (!c->wait_status || !*reinterpret_cast<volatile int*>(c->wait_status)) return JH_OK;
    *reinterpret_cast<volatile int*>(c->wait_status) = 0;
    if (c->attn_sync) {
        hipError_t e = hipMemsetAsync(c->attn_sync, 0, jh::kAttnSyncSlots * sizeof(int), c->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
        if (e != hipSuccess) return hip_fail(c, e, "resetting the in-launch synchronisation state");
    }
    return fail(c, JH_ERR_TIMEOUT,
                std::string(op) + ": a launch that waits for its own blocks (jh_qkv_attention_decode, or a "
                                  "split-K jh_quant_matmul) gave up waiting (were other kernels holding the GPU's "
                                  "CUs?); the outputs it could not finish are NaN (attention heads of that call and "
                                  "of the fused calls after it on this context until now; rows of the product). The "
                                  "synchronisation state was reset: the next call runs normally.");
}

int check_act_dtype(jh_ctx* c, const char* op, const char* what, int dt) {
    if (dt != JH_BF16 && dt != JH_F32)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": " + what + " must be bf16 or f32");
    return JH_OK;
}

// KV caches and the rows appended to them may also be f16 (KVCache.Update casts
// f32 keys and values to f16 on a backend that reports dtypes, qwen/cache.go:90-93).
int check_float_dtype(jh_ctx* c, const char* op, const char* what, int dt) {
    if (dt != JH_BF16 && dt != JH_F32 && dt != JH_F16)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": " + what + " must be bf16, f16 or f32");
    return JH_OK;
}

int finish(jh_ctx* c, const jh::Status& s, const char* op) {
    if (s.code != JH_OK) return fail(c, s.code, s.msg);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(c, e, op);
    return JH_OK;
}

// Read-back checks wait for the stream, which a stream under capture cannot do.
int checks_not_capturing(jh_ctx* c, const char* op) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    JH_HIP(c, hipStreamIsCapturing(c->stream, &cs));
    if (cs != hipStreamCaptureStatusNone)
        return fail(c, JH_ERR_INVALID,
                    std::string(op) + ": checks read results back to the host; turn them off (jh_set_checks) "
                                      "while capturing a graph");
    return JH_OK;
}

// With JH_CHECK_INDICES: device int32 indices copied to the host and each
// checked against [0, limit) before anything is launched.
int check_indices(jh_ctx* c, const char* op, const int32_t* idx, int64_t n, int64_t limit, const char* what) {
    if (!(c->checks & JH_CHECK_INDICES) || n <= 0) return JH_OK;
    if (int r = checks_not_capturing(c, op)) return r;
    std::vector<int32_t> h((size_t)n);
    JH_HIP(c, hipMemcpyAsync(h.data(), idx, h.size() * sizeof(int32_t), hipMemcpyDeviceToHost, c->stream));
    JH_HIP(c, hipStreamSynchronize(c->stream));
    for (size_t i = 0; i < h.size(); i++)
        if (h[i] < 0 || h[i] >= limit)
            return fail(c, JH_ERR_INVALID, std::string(op) + ": " + what + " " + std::to_string(h[i]) + " at " +
                                               std::to_string(i) + " outside [0, " + std::to_string(limit) + ")");
    return JH_OK;
}

// Counts the NaN/Inf among n values of a float type on the device: count and
// the first index (n when none). Waits for the stream.
int count_nonfinite(jh_ctx* c, const char* op, const void* p, int dt, int64_t n, int64_t* count, int64_t* first) {
    if (int r = checks_not_capturing(c, op)) return r;
    if (!c->check_buf) {
        void* b = nullptr;
        if (hipMalloc(&b, 2 * sizeof(unsigned long long)) != hipSuccess) {
            (void)hipGetLastError();
            return fail(c, JH_ERR_OOM, std::string(op) + ": no room for the check counters");
        }
        c->check_buf = static_cast<unsigned long long*>(b);
    }
    const unsigned long long init[2] = {0ull, (unsigned long long)n};
    unsigned long long res[2] = {0ull, 0ull};
    JH_HIP(c, hipMemcpyAsync(c->check_buf, init, sizeof(init), hipMemcpyHostToDevice, c->stream));
    if (int r = finish(c, jh::launch_nonfinite(p, dt, n, c->check_buf, c->stream), "nonfinite_kernel")) return r;
    JH_HIP(c, hipMemcpyAsync(res, c->check_buf, sizeof(res), hipMemcpyDeviceToHost, c->stream));
    JH_HIP(c, hipStreamSynchronize(c->stream));
    *count = (int64_t)res[0];
    *first = (int64_t)res[1];
    return JH_OK;
}

// With JH_CHECK_VALUES, an operator's result is counted for NaN/Inf after it
// runs, as JANIS_GGML_CHECK reads every fp32 result back (ggml/ggml.go:622-677);
// any found is JH_ERR_NONFINITE, naming the operator, the count and the first
// index. The reference exits the process there; here the caller decides.
int check_values(jh_ctx* c, const char* op, const void* y, int dt, int64_t n) {
    if (!(c->checks & JH_CHECK_VALUES) || n <= 0) return JH_OK;
    int64_t bad = 0, first = 0;
    if (int r = count_nonfinite(c, op, y, dt, n, &bad, &first)) return r;
    if (bad)
        return fail(c, JH_ERR_NONFINITE, std::string(op) + ": " + std::to_string(bad) + " of " + std::to_string(n) +
                                             " values NaN/Inf in the result, the first at index " +
                                             std::to_string(first));
    return JH_OK;
}

}  // namespace

namespace {

int check_attention(jh_ctx* c, const char* op, const void* qkv, jh_dtype qkv_dtype, int64_t n_heads,
                    int64_t n_kv_heads, int64_t head_dim, const void* q_norm_w, const void* k_norm_w,
                    jh_dtype w_dtype, int64_t pos, const void* k_cache, const void* v_cache, jh_dtype cache_dtype,
                    int64_t capacity, const void* out, jh_dtype out_dtype) {
    if (int r = check_act_dtype(c, op, "qkv", qkv_dtype)) return r;
    if (int r = check_act_dtype(c, op, "out", out_dtype)) return r;
    if (head_dim != 128) return fail(c, JH_ERR_UNSUPPORTED, std::string(op) + ": head_dim must be 128");
    if (cache_dtype != JH_BF16 && cache_dtype != JH_F16)
        return fail(c, JH_ERR_UNSUPPORTED, std::string(op) + ": the caches must be bf16 or f16");
    if (n_kv_heads <= 0 || n_heads <= 0 || n_heads % n_kv_heads || n_heads > 65536)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": bad head counts");
    const int64_t G = n_heads / n_kv_heads;
    if (G != 1 && G != 2 && G != 4 && G != 8)
        return fail(c, JH_ERR_UNSUPPORTED, std::string(op) + ": n_heads / n_kv_heads must be 1, 2, 4 or 8");
    if ((q_norm_w || k_norm_w) && w_dtype != JH_BF16 && w_dtype != JH_F16 && w_dtype != JH_F32)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": norm weights must be bf16, f16 or f32");
    if (pos < 0 || pos >= capacity || capacity > 0x7fffffff)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": pos " + std::to_string(pos) + " outside the cache capacity " +
                                           std::to_string(capacity));
    if (!qkv || !out || !k_cache || !v_cache || !aligned16(k_cache) || !aligned16(v_cache))
        return fail(c, JH_ERR_INVALID, std::string(op) + ": null pointer, or caches not 16-byte aligned");
    return JH_OK;
}

}  // namespace

extern "C" {

const char* jh_version(void) { return "janis-hip-gfx950 0.1.0"; }

int jh_create(int device, jh_ctx** out) {
    g_create_error.clear();
    if (!out) {
        g_create_error = "jh_create: out is NULL";
        return JH_ERR_INVALID;
    }
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) {
        g_create_error = std::string("jh_create: no HIP device: ") + hipGetErrorString(e);
        return JH_ERR_HIP;
    }
    if (device < 0 || device >= n) {
        g_create_error = "jh_create: device " + std::to_string(device) + " out of range";
        return JH_ERR_INVALID;
    }
    jh_ctx* c = new jh_ctx();
    c->device = device;
    hipDeviceProp_t prop;
    if ((e = hipSetDevice(device)) != hipSuccess || (e = hipGetDeviceProperties(&prop, device)) != hipSuccess ||
        (e = hipStreamCreateWithFlags(&c->own_stream, hipStreamNonBlocking)) != hipSuccess) {
        g_create_error = std::string("jh_create: ") + hipGetErrorString(e);
        delete c;
        return JH_ERR_HIP;
    }
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        g_create_error = std::string("jh_create: device is ") + prop.gcnArchName +
                         ", this library is built for gfx950 only";
        (void)hipStreamDestroy(c->own_stream);
        delete c;
        return JH_ERR_UNSUPPORTED;
    }
    c->stream = c->own_stream;
    c->num_cus = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
    // the no-allocation entry point's scratch, located once per device now, with
    // the device current (a failure here only disables that entry point)
    c->scratch = scratch_address(device);
    // counters of the in-launch attention merge, after checking on the device
    // that block b of a launch runs on XCD b % 8 (a failure only keeps the
    // merge a launch of its own)
    if (hipMalloc(&c->attn_sync, jh::kAttnSyncSlots * sizeof(int)) == hipSuccess) {
        if (hipMemsetAsync(c->attn_sync, 0, jh::kAttnSyncSlots * sizeof(int), c->own_stream) != hipSuccess ||
            jh::probe_xcd_round_robin(c->attn_sync, c->own_stream) != 8 ||
            hipMemsetAsync(c->attn_sync, 0, jh::kAttnSyncSlots * sizeof(int), c->own_stream) != hipSuccess ||
            hipStreamSynchronize(c->own_stream) != hipSuccess) {
            (void)hipGetLastError();
            (void)hipFree(c->attn_sync);
            c->attn_sync = nullptr;
        }
    } else {
        (void)hipGetLastError();
        c->attn_sync = nullptr;
    }
    // the fused launch's give-up status, in host memory so that reading it after
    // a synchronisation costs no copy (a failure only disables the fused launch)
    if (c->attn_sync) {
        void* st = nullptr;
        if (hipHostMalloc(&st, 64, hipHostMallocDefault) == hipSuccess) {
            std::memset(st, 0, 64);
            c->wait_status = static_cast<int*>(st);
        } else {
            (void)hipGetLastError();
        }
    }
    std::snprintf(c->name, sizeof(c->name), "%s (%s, %d CUs)", prop.name, prop.gcnArchName, c->num_cus);
    *out = c;
    return JH_OK;
}

void jh_destroy(jh_ctx* c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    if (c->own_stream) (void)hipStreamSynchronize(c->own_stream);
    if (c->stream && c->stream != c->own_stream) (void)hipStreamSynchronize(c->stream);
    if (c->ws) (void)hipFree(c->ws);
    for (void* p : c->retired) (void)hipFree(p);
    if (c->check_buf) (void)hipFree(c->check_buf);
    if (c->attn_sync) (void)hipFree(c->attn_sync);
    if (c->wait_status) (void)hipHostFree(c->wait_status);
    if (c->own_stream) (void)hipStreamDestroy(c->own_stream);
    delete c;
}

const char* jh_last_error(const jh_ctx* c) { return c ? c->err.c_str() : g_create_error.c_str(); }

int jh_device_info(jh_ctx* c, char* name, size_t name_len, int* compute_units) {
    if (int r = enter(c)) return r;
    if (name && name_len) {
        std::strncpy(name, c->name, name_len - 1);
        name[name_len - 1] = 0;
    }
    if (compute_units) *compute_units = c->num_cus;
    return JH_OK;
}

int jh_set_stream(jh_ctx* c, void* s) {
    if (int r = enter(c)) return r;
    c->stream = s ? static_cast<hipStream_t>(s) : c->own_stream;
    // The in-launch merges rely on workgroups being dealt to the XCDs
    // round-robin, which jh_create checked on the context's own stream; a stream
    // restricted to a subset of the CUs (hipExtStreamCreateWithCUMask) breaks
    // it, so such a stream runs the merges as launches of their own.
    c->stream_xcd_ok = true;
    if (c->stream != c->own_stream) {
        std::vector<uint32_t> mask((size_t)(c->num_cus + 31) / 32, 0u);
        if (hipExtStreamGetCUMask(c->stream, (uint32_t)mask.size(), mask.data()) != hipSuccess) {
            (void)hipGetLastError();
            c->stream_xcd_ok = false;
        } else {
            for (int cu = 0; cu < c->num_cus; cu++)
                if (!((mask[(size_t)cu / 32] >> (cu % 32)) & 1u)) c->stream_xcd_ok = false;
        }
    }
    return JH_OK;
}

int jh_set_wait_limit(jh_ctx* c, int64_t polls) {
    if (int r = enter(c)) return r;
    if (polls < 0 || polls > 0x7fffffff)
        return fail(c, JH_ERR_INVALID, "jh_set_wait_limit: polls must be in [0, 2^31)");
    c->wait_polls = (uint32_t)polls;
    return JH_OK;
}

void* jh_get_stream(const jh_ctx* c) { return c ? static_cast<void*>(c->stream) : nullptr; }

int jh_set_checks(jh_ctx* c, int flags) {
    if (int r = enter(c)) return r;
    if (flags & ~(JH_CHECK_INDICES | JH_CHECK_VALUES))
        return fail(c, JH_ERR_INVALID, "jh_set_checks: unknown check flags " + std::to_string(flags));
    c->checks = flags;
    return JH_OK;
}

int jh_check_finite(jh_ctx* c, const void* x, jh_dtype dtype, int64_t n, int64_t* count, int64_t* first) {
    if (int r = enter(c)) return r;
    const char* op = "jh_check_finite";
    if (dtype != JH_F32 && dtype != JH_BF16 && dtype != JH_F16)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": dtype must be f32, bf16 or f16");
    if (n < 0 || !count || !first) return fail(c, JH_ERR_INVALID, std::string(op) + ": bad arguments");
    *count = 0;
    *first = n;
    if (n == 0) return JH_OK;
    if (!x) return fail(c, JH_ERR_INVALID, std::string(op) + ": null pointer");
    return count_nonfinite(c, op, x, dtype, n, count, first);
}

int jh_sync(jh_ctx* c) {
    if (int r = enter(c)) return r;
    JH_HIP(c, hipStreamSynchronize(c->stream));
    return check_wait_status(c, "jh_sync");
}

int jh_alloc(jh_ctx* c, size_t bytes, void** out) {
    if (int r = enter(c)) return r;
    if (!out) return fail(c, JH_ERR_INVALID, "jh_alloc: out is NULL");
    *out = nullptr;
    if (bytes == 0) bytes = 1;
    hipError_t e = hipMalloc(out, bytes);
    if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) {
        (void)hipGetLastError();
        return fail(c, JH_ERR_OOM, "jh_alloc: out of device memory for " + std::to_string(bytes) + " bytes");
    }
    if (e != hipSuccess) return hip_fail(c, e, "hipMalloc");
    return JH_OK;
}

int jh_free(jh_ctx* c, void* p) {
    if (int r = enter(c)) return r;
    if (!p) return JH_OK;
    JH_HIP(c, hipFree(p));
    return JH_OK;
}

int jh_h2d(jh_ctx* c, void* dst, const void* src, size_t bytes) {
    if (int r = enter(c)) return r;
    if (bytes == 0) return JH_OK;
    if (!dst || !src) return fail(c, JH_ERR_INVALID, "jh_h2d: null pointer");
    JH_HIP(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream));
    JH_HIP(c, hipStreamSynchronize(c->stream));
    return JH_OK;
}

int jh_d2h(jh_ctx* c, void* dst, const void* src, size_t bytes) {
    if (int r = enter(c)) return r;
    if (bytes == 0) return JH_OK;
    if (!dst || !src) return fail(c, JH_ERR_INVALID, "jh_d2h: null pointer");
    JH_HIP(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream));
    JH_HIP(c, hipStreamSynchronize(c->stream));
    return check_wait_status(c, "jh_d2h");
}

int jh_dequantize(jh_ctx* c, const uint32_t* w, const void* scales, const void* biases,
                  jh_dtype sb_dtype, int64_t rows, int64_t in_features, int group_size, int bits,
                  void* out, jh_dtype out_dtype) {
    if (int r = enter(c)) return r;
    if (int r = check_quant(c, "jh_dequantize", w, scales, biases, sb_dtype, rows, in_features,
                            group_size, bits))
        return r;
    if (out_dtype != JH_F32 && out_dtype != JH_BF16)
        return fail(c, JH_ERR_INVALID, "jh_dequantize: out_dtype must be f32 or bf16");
    if (rows == 0) return JH_OK;
    if (!out || !aligned16(out)) return fail(c, JH_ERR_INVALID, "jh_dequantize: out must be 16-byte aligned");
    jh::QuantMatrix m{w, scales, biases, sb_dtype, rows, in_features, group_size, bits};
    if (int r = finish(c, jh::launch_dequantize(m, out, out_dtype, c->stream), "dequant_kernel")) return r;
    return check_values(c, "jh_dequantize", out, out_dtype, rows * in_features);
}

int jh_quant_matmul(jh_ctx* c, const void* x, jh_dtype x_dtype, int64_t rows, const uint32_t* w,
                    const void* scales, const void* biases, jh_dtype sb_dtype, int64_t out_features,
                    int64_t in_features, int transpose, int group_size, int bits, void* y,
                    jh_dtype y_dtype) {
    if (int r = enter(c)) return r;
    const char* op = "jh_quant_matmul";
    if (int r = check_quant(c, op, w, scales, biases, sb_dtype, out_features, in_features, group_size, bits))
        return r;
    if (int r = check_act_dtype(c, op, "x", x_dtype)) return r;
    if (int r = check_act_dtype(c, op, "y", y_dtype)) return r;
    if (rows < 0) return fail(c, JH_ERR_INVALID, "jh_quant_matmul: rows < 0");
    jh::QuantMatrix m{w, scales, biases, sb_dtype, out_features, in_features, group_size, bits};
    if (!transpose) {
        // MatMul(x, Dequantize(w)) (cpu/cpu_misc.go:233-236): x [rows, out_features],
        // y [rows, in_features]
        if (rows == 0 || in_features == 0) return JH_OK;
        if (!x || !y || (out_features > 0 && !w)) return fail(c, JH_ERR_INVALID, std::string(op) + ": null pointer");
        if (rows > 0x7fffffff) return fail(c, JH_ERR_UNSUPPORTED, std::string(op) + ": too many rows");
        if (int r = finish(c, jh::launch_quant_matmul_t(m, x, x_dtype, rows, y, y_dtype, nullptr, 1, 1, 1, c->stream),
                           "qmt"))
            return r;
        return check_values(c, op, y, y_dtype, rows * in_features);
    }
    if (rows == 0 || out_features == 0) return JH_OK;
    if (!x || !y || !aligned16(x) || !aligned16(y))
        return fail(c, JH_ERR_INVALID, "jh_quant_matmul: x and y must be non-null and 16-byte aligned");
    int r;
    if (rows == 1)
        r = finish(c, jh::launch_qmv(m, x, x_dtype, y, y_dtype, c->num_cus, c->stream), "qmv");
    else if (jh::qmv_rows_ok(m, rows, x_dtype))
        r = finish(c, jh::launch_qmv_rows(m, x, x_dtype, rows, y, y_dtype, c->num_cus, c->stream), "qmv_rows");
    else {
        const jh::InLaunchSync sy = qmm_sync(c);
        if (sy.counters)
            if (int e = check_wait_status(c, op)) return e;
        const size_t need = jh::qmm_workspace_bytes(m, rows, x_dtype, y_dtype, c->num_cus, sy.counters != nullptr);
        if (need)
            if (int e = ensure_workspace(c, need, op)) return e;
        r = finish(c, jh::launch_qmm(m, x, x_dtype, rows, y, y_dtype, c->num_cus, c->stream, c->ws, sy), "qmm");
    }
    if (r) return r;
    return check_values(c, op, y, y_dtype, rows * out_features);
}

int jh_quant_matvec_fused(jh_ctx* c, jh_prologue pro, const void* x, jh_dtype x_dtype, const void* norm_w,
                          jh_dtype norm_w_dtype, float eps, const uint32_t* w, const void* scales,
                          const void* biases, jh_dtype sb_dtype, int64_t out_features, int64_t in_features,
                          int group_size, int bits, jh_epilogue epi, const float* resid, void* y,
                          jh_dtype y_dtype, float* norm_stats, void* norm_out) {
    if (int r = enter(c)) return r;
    const char* op = "jh_quant_matvec_fused";
    if (pro != JH_PRO_NONE && pro != JH_PRO_RMSNORM && pro != JH_PRO_SILU_MUL && pro != JH_PRO_NORMED)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": unknown prologue");
    if (epi != JH_EPI_STORE && epi != JH_EPI_RESID && epi != JH_EPI_SWIGLU && epi != JH_EPI_RESID_NORM)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": unknown epilogue");
    if (epi == JH_EPI_RESID_NORM && (pro == JH_PRO_NORMED || pro == JH_PRO_RMSNORM))
        return fail(c, JH_ERR_UNSUPPORTED,
                    std::string(op) + ": a split-norm epilogue cannot follow a norm prologue (one norm_w, one stats)");
    if ((pro == JH_PRO_NORMED || epi == JH_EPI_RESID_NORM) && (!norm_stats || !aligned16(norm_stats)))
        return fail(c, JH_ERR_INVALID, std::string(op) + ": the split norm needs 16-byte aligned norm_stats");
    if (epi == JH_EPI_RESID_NORM && (!norm_out || !norm_w))
        return fail(c, JH_ERR_INVALID, std::string(op) + ": JH_EPI_RESID_NORM needs norm_w and norm_out");
    if (pro == JH_PRO_NORMED && x_dtype != JH_BF16)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": JH_PRO_NORMED takes the bf16 norm_out");
    if (out_features < 0 || (epi == JH_EPI_SWIGLU && out_features > ((int64_t)1 << 40)))
        return fail(c, JH_ERR_INVALID, std::string(op) + ": bad out_features");
    const int64_t w_rows = epi == JH_EPI_SWIGLU ? 2 * out_features : out_features;
    if (int r = check_quant(c, op, w, scales, biases, sb_dtype, w_rows, in_features, group_size, bits)) return r;
    if (int r = check_act_dtype(c, op, "x", x_dtype)) return r;
    if (int r = check_act_dtype(c, op, "y", y_dtype)) return r;
    if ((pro == JH_PRO_RMSNORM || epi == JH_EPI_RESID_NORM) && norm_w_dtype != JH_BF16 && norm_w_dtype != JH_F16 &&
        norm_w_dtype != JH_F32)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": norm weight must be bf16, f16 or f32");
    if ((epi == JH_EPI_RESID || epi == JH_EPI_RESID_NORM) && (y_dtype != JH_F32 || !resid))
        return fail(c, JH_ERR_INVALID, std::string(op) + ": the residual add needs resid and writes fp32 (y_dtype JH_F32)");
    if (out_features == 0) return JH_OK;
    if (!x || !y || !aligned16(x) || !aligned16(y) || (pro == JH_PRO_RMSNORM && (!norm_w || !aligned16(norm_w))))
        return fail(c, JH_ERR_INVALID, std::string(op) + ": x, y (and norm_w) must be non-null and 16-byte aligned");
    jh::QuantMatrix m{w, scales, biases, sb_dtype, w_rows, in_features, group_size, bits};
    const size_t need = jh::qmv_fused_workspace_bytes(m, (int)pro, x_dtype, norm_w_dtype, (int)epi, y_dtype);
    if (need)
        if (int r = ensure_workspace(c, need, op)) return r;
    jh::NormSplit ns;
    ns.stats = norm_stats;
    ns.out = static_cast<uint16_t*>(norm_out);
    if (int r = finish(c, jh::launch_qmv_fused(m, (int)pro, x, x_dtype, norm_w, norm_w_dtype, eps, (int)epi, resid, y,
                                          y_dtype, ns, c->num_cus, c->stream, c->ws),
                  op)) return r;
    return check_values(c, op, y, y_dtype, out_features);
}

int jh_norm_prepare(jh_ctx* c, const void* x, jh_dtype x_dtype, int64_t d, const void* norm_w, jh_dtype norm_w_dtype,
                    void* norm_out, float* norm_stats) {
    if (int r = enter(c)) return r;
    const char* op = "jh_norm_prepare";
    if (int r = check_act_dtype(c, op, "x", x_dtype)) return r;
    if (norm_w_dtype != JH_BF16 && norm_w_dtype != JH_F16 && norm_w_dtype != JH_F32)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": norm weight must be bf16, f16 or f32");
    if (d <= 0) return fail(c, JH_ERR_INVALID, std::string(op) + ": d <= 0");
    if (!x || !norm_w || !norm_out || !norm_stats) return fail(c, JH_ERR_INVALID, std::string(op) + ": null pointer");
    return finish(c, jh::launch_norm_prepare(x, x_dtype, d, norm_w, norm_w_dtype, static_cast<uint16_t*>(norm_out),
                                             norm_stats, c->stream),
                  op);
}

int jh_embed_norm_prepare(jh_ctx* c, const int32_t* ids, const uint32_t* w, const void* scales, const void* biases,
                          jh_dtype sb_dtype, int64_t vocab, int64_t dims, int group_size, int bits, const void* norm_w,
                          jh_dtype norm_w_dtype, float* h, void* norm_out, float* norm_stats, int rope_dims,
                          float rope_base, float rope_scale, int64_t pos, float* rope_cs) {
    if (int r = enter(c)) return r;
    const char* op = "jh_embed_norm_prepare";
    if (int r = check_quant(c, op, w, scales, biases, sb_dtype, vocab, dims, group_size, bits)) return r;
    if (norm_w_dtype != JH_BF16 && norm_w_dtype != JH_F16 && norm_w_dtype != JH_F32)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": norm weight must be bf16, f16 or f32");
    if (vocab <= 0 || dims <= 0) return fail(c, JH_ERR_INVALID, std::string(op) + ": empty table");
    if (!ids || !norm_w || !h || !norm_out || !norm_stats)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": null pointer");
    if (rope_cs && (rope_dims <= 0 || (rope_dims & 1) || rope_dims > 65536 || pos < 0))
        return fail(c, JH_ERR_INVALID, std::string(op) + ": bad RoPE dims or position");
    if (int r = check_indices(c, op, ids, 1, vocab, "id")) return r;
    jh::QuantMatrix m{w, scales, biases, sb_dtype, vocab, dims, group_size, bits};
    return finish(c, jh::launch_embed_norm(ids, m, norm_w, norm_w_dtype, h, static_cast<uint16_t*>(norm_out),
                                           norm_stats, rope_dims, rope_base, rope_scale, pos, rope_cs, c->stream),
                  op);
}

int jh_gather_quant_matmul(jh_ctx* c, const void* x, jh_dtype x_dtype, int64_t n_lead,
                           int64_t a_vectors, const uint32_t* w, const void* scales,
                           const void* biases, jh_dtype sb_dtype, int64_t n_experts,
                           int64_t out_features, int64_t in_features, const int32_t* rhs_indices,
                           int64_t k_slots, int transpose, int group_size, int bits, void* y,
                           jh_dtype y_dtype) {
    if (int r = enter(c)) return r;
    const char* op = "jh_gather_quant_matmul";
    if (int r = check_quant(c, op, w, scales, biases, sb_dtype, out_features, in_features,
                            group_size, bits))
        return r;
    if (int r = check_act_dtype(c, op, "x", x_dtype)) return r;
    if (int r = check_act_dtype(c, op, "y", y_dtype)) return r;
    if (n_lead < 0 || k_slots < 0 || n_experts <= 0)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": bad n_lead / k_slots / n_experts");
    if (a_vectors != 1 && a_vectors != k_slots)
        return fail(c, JH_ERR_INVALID,
                    std::string(op) + ": a_vectors must be 1 or k_slots (x is [lead, A, 1, in])");
    const int64_t n_pairs = n_lead * k_slots;
    if (n_pairs == 0 || out_features == 0) return JH_OK;
    if (n_pairs > (int64_t)1 << 30) return fail(c, JH_ERR_UNSUPPORTED, std::string(op) + ": too many slots");
    if (!x || !y || !rhs_indices || !aligned16(x) || !aligned16(y))
        return fail(c, JH_ERR_INVALID, std::string(op) + ": null or unaligned x / y / indices");
    if (int r = check_indices(c, op, rhs_indices, n_pairs, n_experts, "expert index")) return r;
    if (!transpose) {
        // per slot MatMul(x_slot, Dequantize(W_e)) (cpu/cpu_misc.go:224 with
        // :233-236): x [n_lead, a_vectors, out_features], y [n_pairs, in_features]
        if (n_pairs > 0x7fffffff) return fail(c, JH_ERR_UNSUPPORTED, std::string(op) + ": too many slots");
        jh::QuantMatrix m{w, scales, biases, sb_dtype, out_features, in_features, group_size, bits};
        if (int r = finish(c, jh::launch_quant_matmul_t(m, x, x_dtype, n_pairs, y, y_dtype, rhs_indices, n_experts,
                                                        k_slots, a_vectors, c->stream),
                           "qmt"))
            return r;
        return check_values(c, op, y, y_dtype, n_pairs * in_features);
    }
    jh::GatherArgs a;
    a.m = jh::QuantMatrix{w, scales, biases, sb_dtype, out_features, in_features, group_size, bits};
    a.n_experts = n_experts;
    a.x = x;
    a.x_dtype = x_dtype;
    a.n_lead = n_lead;
    a.a_vectors = a_vectors;
    a.k_slots = k_slots;
    a.idx = rhs_indices;
    a.y = y;
    a.y_dtype = y_dtype;
    a.workspace = nullptr;
    if (jh::gather_uses_workspace(a)) {
        if (int r = ensure_workspace(c, jh::gather_workspace_bytes(n_experts, n_pairs), op)) return r;
        a.workspace = c->ws;
    }
    if (int r = finish(c, jh::launch_gather(a, c->num_cus, c->stream), "gather")) return r;
    return check_values(c, op, y, y_dtype, n_pairs * out_features);
}

int jh_rms_norm(jh_ctx* c, const void* x, jh_dtype x_dtype, int64_t rows, int64_t d, const void* w,
                jh_dtype w_dtype, float eps, void* out, jh_dtype out_dtype) {
    if (int r = enter(c)) return r;
    const char* op = "jh_rms_norm";
    if (int r = check_act_dtype(c, op, "x", x_dtype)) return r;
    if (int r = check_act_dtype(c, op, "out", out_dtype)) return r;
    if (w_dtype != JH_BF16 && w_dtype != JH_F16 && w_dtype != JH_F32)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": weight must be bf16, f16 or f32");
    if (rows < 0 || d <= 0) return fail(c, JH_ERR_INVALID, std::string(op) + ": bad shape");
    if (rows == 0) return JH_OK;
    if (!x || !w || !out) return fail(c, JH_ERR_INVALID, std::string(op) + ": null pointer");
    if (int r = finish(c, jh::launch_rms_norm(x, x_dtype, w, w_dtype, eps, out, out_dtype, rows, d, c->stream), op)) return r;
    return check_values(c, op, out, out_dtype, rows * d);
}

int jh_rope(jh_ctx* c, const void* x, jh_dtype x_dtype, int64_t rows, int64_t L, int64_t D, int dims,
            int traditional, float base, float scale, int64_t offset, const float* freqs, void* out,
            jh_dtype out_dtype) {
    if (int r = enter(c)) return r;
    const char* op = "jh_rope";
    if (int r = check_act_dtype(c, op, "x", x_dtype)) return r;
    if (int r = check_act_dtype(c, op, "out", out_dtype)) return r;
    if (rows < 0 || L <= 0 || D <= 0 || dims <= 0 || dims > D || (dims & 1) || offset < 0)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": bad shape (need 0 < dims <= D, dims even)");
    if (rows == 0) return JH_OK;
    if (!x || !out) return fail(c, JH_ERR_INVALID, std::string(op) + ": null pointer");
    if (int r = finish(c, jh::launch_rope(x, x_dtype, out, out_dtype, rows, L, D, dims, traditional != 0, base, scale,
                                     offset, freqs, c->stream),
                  op)) return r;
    return check_values(c, op, out, out_dtype, rows * D);
}

int jh_sdpa(jh_ctx* c, const void* q, jh_dtype q_dtype, const void* k, const void* v, jh_dtype kv_dtype, int64_t B,
            int64_t Hq, int64_t Hk, int64_t Lq, int64_t Lk, int64_t kv_capacity, int64_t Dh, float scale, int causal,
            void* out, jh_dtype out_dtype) {
    if (int r = enter(c)) return r;
    const char* op = "jh_sdpa";
    if (int r = check_act_dtype(c, op, "q", q_dtype)) return r;
    if (int r = check_float_dtype(c, op, "k/v", kv_dtype)) return r;
    if (int r = check_act_dtype(c, op, "out", out_dtype)) return r;
    if (B < 0 || Hq <= 0 || Hk <= 0 || Hq % Hk || Lq < 0 || Lk < 0 || kv_capacity < Lk || Dh <= 0)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": bad shape (Hq must be a multiple of Hk, capacity >= Lk)");
    if (B * Hq * Lq == 0) return JH_OK;
    if (B * Hq * Lq > 0x7fffffff || Lk > 0x7fffffff || kv_capacity > 0x7fffffff)
        return fail(c, JH_ERR_UNSUPPORTED, std::string(op) + ": too large");
    if (!q || !out || (Lk > 0 && (!k || !v))) return fail(c, JH_ERR_INVALID, std::string(op) + ": null pointer");
    const bool fast = jh::sdpa_decode_ok(q_dtype, kv_dtype, Hq, Hk, Lq, Dh);
    if (fast && (!aligned16(k) || !aligned16(v)))
        return fail(c, JH_ERR_INVALID, std::string(op) + ": k and v must be 16-byte aligned");
    const size_t need = jh::sdpa_workspace_bytes(q_dtype, kv_dtype, B, Hq, Hk, Lq, Lk, Dh, c->num_cus);
    if (need)
        if (int r = ensure_workspace(c, need, op)) return r;
    if (int r = finish(c, jh::launch_sdpa(q, q_dtype, k, v, kv_dtype, out, out_dtype, B, Hq, Hk, Lq, Lk, kv_capacity, Dh,
                                     scale, causal != 0, c->ws, c->num_cus, c->stream),
                  op)) return r;
    return check_values(c, op, out, out_dtype, B * Hq * Lq * Dh);
}

int jh_elementwise(jh_ctx* c, jh_op opk, const void* a, jh_dtype a_dtype, const void* b, jh_dtype b_dtype, int64_t n,
                   void* out, jh_dtype out_dtype) {
    if (int r = enter(c)) return r;
    const char* op = "jh_elementwise";
    if (opk != JH_OP_ADD && opk != JH_OP_MUL && opk != JH_OP_SILU && opk != JH_OP_SILU_MUL)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": unknown operator");
    if (int r = check_act_dtype(c, op, "a", a_dtype)) return r;
    if (opk != JH_OP_SILU)
        if (int r = check_act_dtype(c, op, "b", b_dtype)) return r;
    if (int r = check_act_dtype(c, op, "out", out_dtype)) return r;
    if (n < 0) return fail(c, JH_ERR_INVALID, std::string(op) + ": n < 0");
    if (n == 0) return JH_OK;
    if (!a || !out || (opk != JH_OP_SILU && !b)) return fail(c, JH_ERR_INVALID, std::string(op) + ": null pointer");
    if (int r = finish(c, jh::launch_elementwise((int)opk, a, a_dtype, b, b_dtype, out, out_dtype, n, c->stream), op)) return r;
    return check_values(c, op, out, out_dtype, n);
}

int jh_argmax(jh_ctx* c, const void* x, jh_dtype x_dtype, int64_t rows, int64_t n, int32_t* out) {
    if (int r = enter(c)) return r;
    const char* op = "jh_argmax";
    if (int r = check_act_dtype(c, op, "x", x_dtype)) return r;
    if (rows < 0 || n <= 0) return fail(c, JH_ERR_INVALID, std::string(op) + ": bad shape");
    if (rows == 0) return JH_OK;
    if (rows > 0x7fffffff) return fail(c, JH_ERR_UNSUPPORTED, std::string(op) + ": too many rows");
    if (!x || !out) return fail(c, JH_ERR_INVALID, std::string(op) + ": null pointer");
    if (int r = ensure_workspace(c, jh::argmax_workspace_bytes(rows), op)) return r;
    return finish(c, jh::launch_argmax(x, x_dtype, rows, n, out, c->ws, c->attn_sync, c->stream), op);
}

int jh_qk_norm_rope_append(jh_ctx* c, const void* qkv, jh_dtype qkv_dtype, int64_t n_heads, int64_t n_kv_heads,
                           int64_t head_dim, const void* q_norm_w, const void* k_norm_w, jh_dtype w_dtype, float eps,
                           float rope_base, float rope_scale, int64_t pos, void* k_cache, void* v_cache,
                           jh_dtype cache_dtype, int64_t capacity, void* q_out, jh_dtype q_out_dtype) {
    if (int r = enter(c)) return r;
    const char* op = "jh_qk_norm_rope_append";
    if (int r = check_act_dtype(c, op, "qkv", qkv_dtype)) return r;
    if (int r = check_float_dtype(c, op, "cache", cache_dtype)) return r;
    if (int r = check_act_dtype(c, op, "q_out", q_out_dtype)) return r;
    if (w_dtype != JH_BF16 && w_dtype != JH_F16 && w_dtype != JH_F32)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": norm weights must be bf16, f16 or f32");
    if (head_dim != 128) return fail(c, JH_ERR_UNSUPPORTED, std::string(op) + ": head_dim must be 128");
    if (n_heads <= 0 || n_kv_heads <= 0 || n_heads > 4096 || n_kv_heads > 4096 || pos < 0 || pos >= capacity)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": bad heads, or pos outside the cache capacity");
    if (!qkv || !q_norm_w || !k_norm_w || !k_cache || !v_cache || !q_out)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": null pointer");
    return finish(c, jh::launch_qk_norm_rope_append(qkv, qkv_dtype, (int)n_heads, (int)n_kv_heads, q_norm_w, k_norm_w,
                                                    w_dtype, eps, rope_base, rope_scale, pos, k_cache, v_cache,
                                                    cache_dtype, capacity, q_out, q_out_dtype, c->stream),
                  op);
}

int jh_rope_table(jh_ctx* c, int dims, float base, float scale, int64_t pos, const float* freqs, float* out) {
    if (int r = enter(c)) return r;
    const char* op = "jh_rope_table";
    if (dims <= 0 || (dims & 1) || dims > 65536 || pos < 0)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": bad dims or position");
    if (!out) return fail(c, JH_ERR_INVALID, std::string(op) + ": null pointer");
    return finish(c, jh::launch_rope_table(dims, base, scale, pos, freqs, out, c->stream), op);
}


int jh_attention_decode(jh_ctx* c, const void* qkv, jh_dtype qkv_dtype, int64_t n_heads, int64_t n_kv_heads,
                        int64_t head_dim, const void* q_norm_w, const void* k_norm_w, jh_dtype w_dtype, float eps,
                        float rope_base, float rope_scale, const float* rope_cs, int64_t pos, void* k_cache,
                        void* v_cache,
                        jh_dtype cache_dtype, int64_t capacity, float scale, void* out, jh_dtype out_dtype) {
    if (int r = enter(c)) return r;
    const char* op = "jh_attention_decode";
    if (int r = check_attention(c, op, qkv, qkv_dtype, n_heads, n_kv_heads, head_dim, q_norm_w, k_norm_w, w_dtype, pos,
                                k_cache, v_cache, cache_dtype, capacity, out, out_dtype))
        return r;
    const size_t need = jh::attn_decode_workspace_bytes(n_heads, n_kv_heads, pos, c->num_cus);
    if (need)
        if (int r = ensure_workspace(c, need, op)) return r;
    if (int r = finish(c, jh::launch_attn_decode(qkv, qkv_dtype, (int)n_heads, (int)n_kv_heads, q_norm_w, k_norm_w,
                                                 w_dtype, eps, rope_base, rope_scale, rope_cs, pos, k_cache, v_cache,
                                                 cache_dtype, capacity, scale, out, out_dtype, c->ws, c->num_cus,
                                                 c->stream, xcd_sync(c)),
                       op))
        return r;
    return check_values(c, op, out, out_dtype, n_heads * head_dim);
}

int jh_qkv_attention_decode(jh_ctx* c, const void* x, const float* norm_stats, float norm_eps, const uint32_t* w,
                            const void* scales, const void* biases, jh_dtype sb_dtype, int64_t in_features,
                            int group_size, int bits, void* qkv, jh_dtype qkv_dtype, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                            const void* q_norm_w, const void* k_norm_w, jh_dtype w_dtype, float eps, float rope_base,
                            float rope_scale, const float* rope_cs, int64_t pos, void* k_cache, void* v_cache,
                            jh_dtype cache_dtype, int64_t capacity, float scale, void* out, jh_dtype out_dtype) {
    if (int r = enter(c)) return r;
    const char* op = "jh_qkv_attention_decode";
    if (n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 || n_heads % n_kv_heads != 0)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": bad head counts");
    const int64_t rows = (n_heads + 2 * n_kv_heads) * head_dim;
    if (int r = check_quant(c, op, w, scales, biases, sb_dtype, rows, in_features, group_size, bits)) return r;
    if (!x || !aligned16(x) || !norm_stats || !aligned16(norm_stats) || !qkv || !aligned16(qkv))
        return fail(c, JH_ERR_INVALID, std::string(op) + ": x, norm_stats and qkv must be non-null and 16-byte aligned");
    if (qkv_dtype != JH_BF16 && qkv_dtype != JH_F32)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": qkv must be bf16 or f32");
    if (int r = check_attention(c, op, qkv, qkv_dtype, n_heads, n_kv_heads, head_dim, q_norm_w, k_norm_w, w_dtype, pos,
                                k_cache, v_cache, cache_dtype, capacity, out, out_dtype))
        return r;
    const jh::QuantMatrix m{w, scales, biases, sb_dtype, rows, in_features, group_size, bits};
    const size_t need = jh::attn_decode_workspace_bytes(n_heads, n_kv_heads, pos, c->num_cus);
    if (need)
        if (int r = ensure_workspace(c, need, op)) return r;
    if (c->wait_status && jh::qkv_attn_ok(m, n_heads, n_kv_heads, xcd_sync(c), c->num_cus)) {
        // an earlier fused call's wait that gave up is reported as soon as the
        // host can see it
        if (int r = check_wait_status(c, op)) return r;
        const jh::Status st = jh::launch_qkv_attn(m, static_cast<const uint16_t*>(x), const_cast<float*>(norm_stats),
                                                  norm_eps, qkv, (int)qkv_dtype, (int)n_heads, (int)n_kv_heads,
                                                  q_norm_w, k_norm_w, w_dtype, eps, rope_base, rope_scale, rope_cs, pos,
                                                  k_cache, v_cache, cache_dtype, capacity, scale, out, out_dtype, c->ws,
                                                  c->num_cus, c->stream, xcd_sync(c), c->wait_polls, c->wait_status);
        if (st.code != JH_ERR_UNSUPPORTED) {
            if (int r = finish(c, st, op)) return r;
            return check_values(c, op, out, out_dtype, n_heads * head_dim);
        }
    }
    // otherwise the two operators it fuses, one after the other
    if (int r = jh_quant_matvec_fused(c, JH_PRO_NORMED, x, JH_BF16, nullptr, JH_BF16, norm_eps, w, scales, biases,
                                      sb_dtype, rows, in_features, group_size, bits, JH_EPI_STORE, nullptr, qkv,
                                      qkv_dtype, const_cast<float*>(norm_stats), nullptr))
        return r;
    return jh_attention_decode(c, qkv, qkv_dtype, n_heads, n_kv_heads, head_dim, q_norm_w, k_norm_w, w_dtype, eps,
                               rope_base, rope_scale, rope_cs, pos, k_cache, v_cache, cache_dtype, capacity, scale, out,
                               out_dtype);
}

int jh_attention_decode_noalloc(jh_ctx* c, const void* qkv, jh_dtype qkv_dtype, int64_t n_heads, int64_t n_kv_heads,
                                int64_t head_dim, const void* q_norm_w, const void* k_norm_w, jh_dtype w_dtype,
                                float eps, float rope_base, float rope_scale, const float* rope_cs, int64_t pos,
                                void* k_cache, void* v_cache, jh_dtype cache_dtype, int64_t capacity, float scale,
                                void* out, jh_dtype out_dtype) {
    if (int r = enter(c)) return r;
    const char* op = "jh_attention_decode_noalloc";
    if (int r = check_attention(c, op, qkv, qkv_dtype, n_heads, n_kv_heads, head_dim, q_norm_w, k_norm_w, w_dtype, pos,
                                k_cache, v_cache, cache_dtype, capacity, out, out_dtype))
        return r;
    if (!c->scratch)
        return fail(c, JH_ERR_HIP, std::string(op) + ": the device scratch array could not be located");
    const size_t need = jh::attn_decode_workspace_bytes(n_heads, n_kv_heads, pos, c->num_cus);
    if (need > kScratchBytes)
        return fail(c, JH_ERR_UNSUPPORTED, std::string(op) + ": needs " + std::to_string(need) +
                                               " bytes of partials, more than the " + std::to_string(kScratchBytes) +
                                               "-byte scratch (use jh_attention_decode)");
    // every split block writes all of its partials before the merge reads them,
    // so the scratch needs no clearing
    if (int r = finish(c, jh::launch_attn_decode(qkv, qkv_dtype, (int)n_heads, (int)n_kv_heads, q_norm_w, k_norm_w,
                                                 w_dtype, eps, rope_base, rope_scale, rope_cs, pos, k_cache, v_cache,
                                                 cache_dtype, capacity, scale, out, out_dtype, c->scratch, c->num_cus,
                                                 c->stream, xcd_sync(c)),
                       op))
        return r;
    return check_values(c, op, out, out_dtype, n_heads * head_dim);
}

int jh_copy_strided(jh_ctx* c, const void* src, jh_dtype src_dtype, int ndim, const int64_t* shape,
                    const int64_t* src_strides, void* dst, jh_dtype dst_dtype, const int64_t* dst_strides) {
    if (int r = enter(c)) return r;
    const char* op = "jh_copy_strided";
    auto is_float = [](int dt) { return dt == JH_F32 || dt == JH_F16 || dt == JH_BF16; };
    if (src_dtype < JH_F32 || src_dtype > JH_U8 || dst_dtype < JH_F32 || dst_dtype > JH_U8)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": unknown dtype");
    if (src_dtype != dst_dtype && !(is_float(src_dtype) && is_float(dst_dtype)))
        return fail(c, JH_ERR_UNSUPPORTED, std::string(op) + ": integer types copy only to themselves");
    if (ndim < 0 || ndim > jh::kMaxCopyDims || (ndim > 0 && (!shape || !src_strides)))
        return fail(c, JH_ERR_INVALID, std::string(op) + ": ndim must be 0.." + std::to_string(jh::kMaxCopyDims));
    int64_t n = 1;
    for (int a = 0; a < ndim; a++) {
        if (shape[a] < 0) return fail(c, JH_ERR_INVALID, std::string(op) + ": negative extent");
        n *= shape[a];
    }
    if (n == 0) return JH_OK;
    if (!src || !dst) return fail(c, JH_ERR_INVALID, std::string(op) + ": null pointer");
    return finish(c, jh::launch_copy_strided(src, src_dtype, ndim, shape, src_strides, dst, dst_dtype, dst_strides,
                                             c->stream),
                  op);
}

int jh_take_rows(jh_ctx* c, const void* table, int64_t row_bytes, int64_t n_rows, const int32_t* ids, int64_t n_ids,
                 void* out) {
    if (int r = enter(c)) return r;
    const char* op = "jh_take_rows";
    if (row_bytes < 0 || n_rows < 0 || n_ids < 0) return fail(c, JH_ERR_INVALID, std::string(op) + ": bad shape");
    if (n_ids == 0 || row_bytes == 0) return JH_OK;
    if (n_ids > 0x7fffffff) return fail(c, JH_ERR_UNSUPPORTED, std::string(op) + ": too many ids");
    if (!table || !ids || !out) return fail(c, JH_ERR_INVALID, std::string(op) + ": null pointer");
    if (int r = check_indices(c, op, ids, n_ids, n_rows, "id")) return r;
    return finish(c, jh::launch_take_rows(table, row_bytes, n_rows, ids, n_ids, out, c->stream), op);
}

int jh_scatter_rows(jh_ctx* c, const void* dst, void* out, int64_t rows, int64_t row_bytes, const int32_t* indices,
                    int64_t n_indices, const void* updates) {
    if (int r = enter(c)) return r;
    const char* op = "jh_scatter_rows";
    if (rows < 0 || row_bytes < 0 || n_indices < 0) return fail(c, JH_ERR_INVALID, std::string(op) + ": bad shape");
    if (rows > 0x7fffffff || n_indices > 0x7fffffff)
        return fail(c, JH_ERR_UNSUPPORTED, std::string(op) + ": more than 2^31 rows");
    if (n_indices > 0 && !indices) return fail(c, JH_ERR_INVALID, std::string(op) + ": null indices");
    // every index is checked before anything is written
    for (int64_t i = 0; i < n_indices; i++)
        if (indices[i] < 0 || indices[i] >= rows)
            return fail(c, JH_ERR_INVALID, std::string(op) + ": index " + std::to_string(indices[i]) + " at " +
                                               std::to_string(i) + " outside [0, " + std::to_string(rows) + ")");
    if (rows == 0 || row_bytes == 0) return JH_OK;
    if (!dst || !out || (n_indices > 0 && !updates)) return fail(c, JH_ERR_INVALID, std::string(op) + ": null pointer");
    if (out != dst)
        JH_HIP(c, hipMemcpyAsync(out, dst, (size_t)(rows * row_bytes), hipMemcpyDeviceToDevice, c->stream));
    // a repeated index keeps its last update (the order the updates are applied
    // in), so each destination row is written once and the launches cannot race
    std::vector<char> seen((size_t)rows, 0);
    jh::ScatterList l;
    l.n = 0;
    for (int64_t i = n_indices - 1; i >= 0; i--) {
        const int32_t r = indices[i];
        if (seen[(size_t)r]) continue;
        seen[(size_t)r] = 1;
        l.dst[l.n] = r;
        l.src[l.n] = (int32_t)i;
        if (++l.n == jh::kScatterBatch) {
            if (int e = finish(c, jh::launch_scatter_rows(l, updates, out, row_bytes, c->stream), op)) return e;
            l.n = 0;
        }
    }
    return finish(c, jh::launch_scatter_rows(l, updates, out, row_bytes, c->stream), op);
}

int jh_kv_append(jh_ctx* c, void* k_cache, void* v_cache, jh_dtype cache_dtype, int64_t BH, int64_t capacity,
                 int64_t pos, const void* k_new, const void* v_new, jh_dtype new_dtype, int64_t L, int64_t Dh) {
    if (int r = enter(c)) return r;
    const char* op = "jh_kv_append";
    if (int r = check_float_dtype(c, op, "cache", cache_dtype)) return r;
    if (int r = check_float_dtype(c, op, "new rows", new_dtype)) return r;
    if (BH < 0 || capacity < 0 || pos < 0 || L < 0 || Dh <= 0 || pos + L > capacity)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": rows " + std::to_string(pos) + ".." +
                                           std::to_string(pos + L) + " do not fit capacity " + std::to_string(capacity));
    if (BH * L == 0) return JH_OK;
    if (!k_cache || !v_cache || !k_new || !v_new) return fail(c, JH_ERR_INVALID, std::string(op) + ": null pointer");
    return finish(c, jh::launch_kv_append(k_cache, v_cache, cache_dtype, k_new, v_new, new_dtype, BH, capacity, pos, L,
                                          Dh, c->stream),
                  op);
}

int jh_moe_route(jh_ctx* c, const void* logits, jh_dtype logits_dtype, int64_t n_tok, int64_t n_experts,
                 int64_t k, int norm_topk, int32_t* rhs_indices, float* scores) {
    if (int r = enter(c)) return r;
    const char* op = "jh_moe_route";
    if (int r = check_act_dtype(c, op, "logits", logits_dtype)) return r;
    if (n_tok < 0 || n_experts <= 0 || k < 0 || k > n_experts)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": need n_tok >= 0 and 0 <= k <= n_experts");
    if (n_tok == 0 || k == 0) return JH_OK;
    if (!logits || !rhs_indices || !scores)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": null logits / indices / scores");
    return finish(c, jh::launch_moe_route(logits, logits_dtype, n_tok, (int)n_experts, (int)k, norm_topk != 0,
                                          rhs_indices, scores, c->stream),
                  "moe_route");
}

int jh_moe_swiglu(jh_ctx* c, const void* x, jh_dtype x_dtype, int64_t n_tok, const uint32_t* w_gate,
                  const void* s_gate, const void* b_gate, const uint32_t* w_up, const void* s_up,
                  const void* b_up, const uint32_t* w_down, const void* s_down, const void* b_down,
                  jh_dtype sb_dtype, int64_t n_experts, int64_t hidden, int64_t intermediate,
                  const int32_t* rhs_indices, const float* scores, int64_t k_slots, int group_size,
                  int bits, void* out, jh_dtype out_dtype) {
    if (int r = enter(c)) return r;
    const char* op = "jh_moe_swiglu";
    if (int r = check_quant(c, op, w_gate, s_gate, b_gate, sb_dtype, intermediate, hidden, group_size, bits))
        return r;
    if (int r = check_quant(c, op, w_up, s_up, b_up, sb_dtype, intermediate, hidden, group_size, bits))
        return r;
    if (int r = check_quant(c, op, w_down, s_down, b_down, sb_dtype, hidden, intermediate, group_size, bits))
        return r;
    if (x_dtype != JH_BF16) return fail(c, JH_ERR_UNSUPPORTED, std::string(op) + ": x must be bf16");
    if (bits != 4) return fail(c, JH_ERR_UNSUPPORTED, std::string(op) + ": only 4-bit expert stacks are fused");
    if (int r = check_act_dtype(c, op, "out", out_dtype)) return r;
    if (n_tok < 0 || k_slots < 0 || n_experts <= 0 || intermediate <= 0)
        return fail(c, JH_ERR_INVALID, std::string(op) + ": bad n_tok / k_slots / n_experts / intermediate");
    const int64_t n_pairs = n_tok * k_slots;
    if (n_tok == 0) return JH_OK;
    if (n_pairs > (int64_t)1 << 30) return fail(c, JH_ERR_UNSUPPORTED, std::string(op) + ": too many slots");
    if (!x || !out || !aligned16(x) || !aligned16(out) || (n_pairs > 0 && (!rhs_indices || !scores)))
        return fail(c, JH_ERR_INVALID, std::string(op) + ": null or unaligned x / out / indices / scores");
    jh::MoeMlpArgs a;
    a.gate = jh::QuantMatrix{w_gate, s_gate, b_gate, sb_dtype, intermediate, hidden, group_size};
    a.up = jh::QuantMatrix{w_up, s_up, b_up, sb_dtype, intermediate, hidden, group_size};
    a.down = jh::QuantMatrix{w_down, s_down, b_down, sb_dtype, hidden, intermediate, group_size};
    a.n_experts = n_experts;
    a.x = x;
    a.n_tok = n_tok;
    a.k_slots = k_slots;
    a.idx = rhs_indices;
    a.scores = scores;
    a.out = out;
    a.out_dtype = out_dtype;
    if (const char* why = jh::moe_unsupported(a))
        return fail(c, JH_ERR_UNSUPPORTED, std::string(op) + ": " + why);
    if (int r = check_indices(c, op, rhs_indices, n_pairs, n_experts, "expert index")) return r;
    if (int r = ensure_workspace(c, jh::moe_workspace_bytes(a), op)) return r;
    if (int r = finish(c, jh::launch_moe_mlp(a, c->ws, c->stream), "moe_swiglu")) return r;
    return check_values(c, op, out, out_dtype, n_tok * hidden);
}

int jh_softmax(jh_ctx* c, const void* x, jh_dtype x_dtype, int64_t outer, int64_t len, int64_t inner, float* y) {
    if (int r = enter(c)) return r;
    const char* op = "jh_softmax";
    if (int r = check_act_dtype(c, op, "x", x_dtype)) return r;
    if (outer < 0 || len < 0 || inner < 0) return fail(c, JH_ERR_INVALID, std::string(op) + ": bad shape");
    if (outer * len * inner == 0) return JH_OK;
    if (!x || !y) return fail(c, JH_ERR_INVALID, std::string(op) + ": null pointer");
    if (int r = finish(c, jh::launch_softmax(x, x_dtype, y, outer, len, inner, c->stream), op)) return r;
    return check_values(c, op, y, JH_F32, outer * len * inner);
}

int jh_mean(jh_ctx* c, const void* x, jh_dtype x_dtype, int64_t outer, int64_t len, int64_t inner, float* y) {
    if (int r = enter(c)) return r;
    const char* op = "jh_mean";
    if (int r = check_act_dtype(c, op, "x", x_dtype)) return r;
    if (outer < 0 || len < 0 || inner < 0) return fail(c, JH_ERR_INVALID, std::string(op) + ": bad shape");
    if (outer * inner == 0) return JH_OK;
    if (!y || (len > 0 && !x)) return fail(c, JH_ERR_INVALID, std::string(op) + ": null pointer");
    if (int r = finish(c, jh::launch_mean(x, x_dtype, y, outer, len, inner, c->stream), op)) return r;
    return check_values(c, op, y, JH_F32, outer * inner);
}

int jh_scalar(jh_ctx* c, jh_scalar_op sop, const void* x, jh_dtype x_dtype, int64_t n, float v, void* y,
              jh_dtype y_dtype) {
    if (int r = enter(c)) return r;
    const char* op = "jh_scalar";
    if (sop != JH_SCALAR_MUL && sop != JH_SCALAR_ADD) return fail(c, JH_ERR_INVALID, std::string(op) + ": unknown op");
    if (int r = check_act_dtype(c, op, "x", x_dtype)) return r;
    if (int r = check_act_dtype(c, op, "y", y_dtype)) return r;
    if (n < 0) return fail(c, JH_ERR_INVALID, std::string(op) + ": n < 0");
    if (n == 0) return JH_OK;
    if (!x || !y) return fail(c, JH_ERR_INVALID, std::string(op) + ": null pointer");
    if (int r = finish(c, jh::launch_scalar((int)sop, x, x_dtype, v, y, y_dtype, n, c->stream), op)) return r;
    return check_values(c, op, y, y_dtype, n);
}

}  // extern "C"
