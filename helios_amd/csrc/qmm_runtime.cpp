// C ABI of libgemma4_qmm (include/gemma4_qmm.h): handles, errors, dispatch.
//
// Mirrors the reference runtime's conventions (native/gemma4_mlx/src/runtime.cc):
// status codes, a thread-local last-error buffer (runtime.cc:46, :116-133), magic
// numbers on handles (runtime.cc:41-45), no exception across the ABI.
#include "gemma4_qmm.h"

#include <hip/hip_runtime.h>

#include <atomic>
#include <climits>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <new>
#include <string>
#include <thread>
#include <vector>

#include "q4_common.h"
#include "q4_kernels.h"

namespace {

constexpr uint64_t kQLinearMagic = 0x47454d3451344c4eULL;  // "GEM4Q4LN"
constexpr int kGreedyMaxRows = 16;  // rows per greedy-head call (decode and verify blocks)
constexpr uint64_t kLoraMagic = 0x47454d344c4f5241ULL;  // "GEM4LORA"
thread_local char g_last_error[512] = "";
// forward path choice: 0 = automatic (q4::use_decode), r > 0 = the GEMM from r rows on
std::atomic<uint32_t> g_gemm_min_rows{0};
// GEMM form: 0 the pre-pass forms where the plan takes them, 1 the bf16 form only
std::atomic<uint32_t> g_gemm_form{0};

// Records the message (truncated to the buffer) and returns status.  The const char*
// forms build no std::string, so they cannot throw: catch blocks use them.
Gemma4Status fail_nothrow(Gemma4Status status, const char* message) noexcept {
    std::snprintf(g_last_error, sizeof(g_last_error), "%s", message);
    return status;
}

Gemma4Status fail(Gemma4Status status, const char* message) noexcept { return fail_nothrow(status, message); }

Gemma4Status fail(Gemma4Status status, const std::string& message) noexcept {
    return fail_nothrow(status, message.c_str());
}

Gemma4Status ok() {
    g_last_error[0] = '\0';
    return GEMMA4_OK;
}

Gemma4Status hip_fail(const char* where, hipError_t e) {
    return fail(GEMMA4_ERR_RUNTIME, std::string(where) + ": " + hipGetErrorName(e) + " (" +
                                        hipGetErrorString(e) + ")");
}

// Per-device stream-ordered memory pool for per-call scratch (the GEMM's group sums
// of x).  Its release threshold is unlimited, so after the first calls allocations
// are served from memory the pool keeps; it is separate from the device's default
// pool, so callers' own allocators are untouched.  Allocations are stream-ordered,
// which keeps forward reentrant across streams.
std::mutex g_pool_mu;
hipMemPool_t g_pools[64] = {};

hipError_t scratch_pool(int device, hipMemPool_t* out) {
    if (device < 0 || device >= 64) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_pool_mu);
    if (g_pools[device] == nullptr) {
        hipMemPoolProps props{};
        props.allocType = hipMemAllocationTypePinned;
        props.handleTypes = hipMemHandleTypeNone;
        props.location.type = hipMemLocationTypeDevice;
        props.location.id = device;
        hipMemPool_t pool = nullptr;
        hipError_t e = hipMemPoolCreate(&pool, &props);
        if (e != hipSuccess) return e;
        uint64_t keep = UINT64_MAX;
        e = hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep);
        if (e != hipSuccess) {
            (void)hipMemPoolDestroy(pool);
            return e;
        }
        g_pools[device] = pool;
    }
    *out = g_pools[device];
    return hipSuccess;
}

// The bf16 GeGLU epilogue's table of gelu over bf16 patterns (5.5 KiB), built
// once per device when its first gate|up pair is created (create synchronizes, so
// every later forward, on any stream, sees it complete).  Kept until the process ends.
std::mutex g_table_mu;
uint16_t* g_gelu_tables[64] = {};

hipError_t gelu_table(int device, const uint16_t** out) {
    if (device < 0 || device >= 64) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_table_mu);
    if (g_gelu_tables[device] == nullptr) {
        uint16_t* t = nullptr;
        hipError_t e = hipMalloc(&t, q4::kGeluTable * sizeof(uint16_t));
        if (e != hipSuccess) return e;
        e = q4::launch_gelu_table(t, nullptr);
        if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
        if (e != hipSuccess) {
            (void)hipFree(t);
            return e;
        }
        g_gelu_tables[device] = t;
    }
    *out = g_gelu_tables[device];
    return hipSuccess;
}

// The allocation-free forward's scratch (gemma4_qlinear_forward_noalloc): one
// file-scope device array, which every GPU the library runs on holds (its own copy,
// at its own address) until the process ends.  In host code `scratch` names a host
// stand-in, not device memory: its device address comes from hipGetSymbolAddress,
// once per device with that device current, and only that address is used.
constexpr size_t kStaticScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[64] = {};

// The current device's address of `scratch` (device must be current).
hipError_t static_scratch(int device, char** out) {
    if (device < 0 || device >= 64) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[device] == nullptr) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (ptr == nullptr) return hipErrorInvalidSymbol;
        g_scratch_ptr[device] = ptr;
    }
    *out = static_cast<char*>(g_scratch_ptr[device]);
    return hipSuccess;
}

// Device memory kept per (device, stream) for the scratch of the calls on that stream.
// Work on one stream runs in order, so consecutive calls can reuse it; `mu` is held
// for a whole call (its scratch and its launches), so calls from several host threads
// on one stream cannot interleave their launches.  It grows by allocating a larger
// buffer when a call is not being captured into a graph.  An outgrown buffer that a
// capture took pieces of is kept (a graph captured earlier may still use it) until
// gemma4_qmm_release_scratch; one no capture used is freed once the stream is idle.  A
// stream-ordered pool allocation per call (and, under capture, an allocation node per
// call in the graph) cost 5-10 us per forward on the GPU: k_proj 2048x3840 at 512 rows,
// split four ways, 31 us per forward in a graph against 22 us with the workspace.
struct StreamWorkspace {
    int device = -1;
    hipStream_t stream = nullptr;
    std::thread::id thread;  // hipStreamPerThread: a different stream in every thread
    char* buf = nullptr;
    size_t cap = 0;
    bool buf_captured = false;    // a graph capture took pieces of buf
    std::vector<char*> retired;  // outgrown buffers that captures used
    std::mutex mu;
};
std::mutex g_ws_mu;
std::vector<std::unique_ptr<StreamWorkspace>> g_ws;


StreamWorkspace* stream_workspace(int device, hipStream_t stream) {
    const std::thread::id thread = stream == hipStreamPerThread ? std::this_thread::get_id() : std::thread::id();
    std::lock_guard<std::mutex> lock(g_ws_mu);
    for (auto& w : g_ws)
        if (w->device == device && w->stream == stream && w->thread == thread) return w.get();
    g_ws.push_back(std::make_unique<StreamWorkspace>());
    g_ws.back()->device = device;
    g_ws.back()->stream = stream;
    g_ws.back()->thread = thread;
    return g_ws.back().get();
}

// Device memory one call borrows for its kernels' scratch (the GEMM's group sums and
// split-K partials, the greedy head's keys, LoRA's x.A^T): consecutive 256-byte-aligned
// pieces of the stream's workspace, or, for the allocation-free entry point, of
// `scratch`.  A call captured into a graph whose stream workspace is too small takes
// stream-ordered allocations from the private pool instead, released on the same
// stream after the launches (allocation nodes of the graph).
struct Scratch {
    hipStream_t stream = nullptr;
    int device = 0;
    bool fixed = false;  // pieces of `scratch`: no allocation and nothing to release
    char* base = nullptr;
    size_t cap = 0, used = 0;
    StreamWorkspace* ws = nullptr;  // the stream's workspace (not fixed)
    std::unique_lock<std::mutex> ws_lock;
    void* owned[2] = {};
    int n_owned = 0;

    // bytes still available (fixed mode; unlimited otherwise)
    size_t room() const { return fixed ? cap - used : ~(size_t)0; }

    hipError_t take(size_t bytes, void** out) {
        *out = nullptr;
        if (bytes == 0) return hipSuccess;
        const size_t need = (bytes + 255) & ~(size_t)255;
        if (fixed) {
            if (need > cap - used) return hipErrorOutOfMemory;
            *out = base + used;
            used += need;
            return hipSuccess;
        }
        if (ws == nullptr) {
            ws = stream_workspace(device, stream);
            ws_lock = std::unique_lock<std::mutex>(ws->mu);
            base = ws->buf;
            cap = ws->cap;
            used = 0;
        }
        hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
        const bool capturing =
            hipStreamIsCapturing(stream, &capture) != hipSuccess || capture != hipStreamCaptureStatusNone;
        if (need <= cap - used) {
            *out = base + used;
            used += need;
            if (capturing) ws->buf_captured = true;
            return hipSuccess;
        }
        if (!capturing) {
            // grow: a new buffer for this and later calls.  Pieces this call took from
            // the old one stay valid (it is released only after this call's launches,
            // see `finish`), as does every graph that used it.  (The pool for the
            // fallback below is made here too, outside any capture.)
            hipMemPool_t pool = nullptr;
            (void)scratch_pool(device, &pool);
            size_t ncap = ws->cap * 2 > need ? ws->cap * 2 : need;
            ncap = (ncap + ((size_t)1 << 20) - 1) & ~(((size_t)1 << 20) - 1);
            char* nb = nullptr;
            if (hipMalloc(&nb, ncap) == hipSuccess) {
                if (ws->buf != nullptr) {
                    if (ws->buf_captured)
                        ws->retired.push_back(ws->buf);
                    else
                        outgrown = ws->buf;
                }
                ws->buf = base = nb;
                ws->cap = cap = ncap;
                ws->buf_captured = false;
                *out = base;
                used = need;
                return hipSuccess;
            }
            (void)hipGetLastError();  // out of memory: fall back to the pool
        }
        if (n_owned == 2) return hipErrorInvalidValue;
        hipMemPool_t pool = nullptr;
        hipError_t e = scratch_pool(device, &pool);
        if (e == hipSuccess) e = hipMallocFromPoolAsync(out, bytes, pool, stream);
        if (e == hipSuccess) owned[n_owned++] = *out;
        return e;
    }

    // queues the release of every pool allocation after the work on the stream
    hipError_t release() {
        hipError_t first = hipSuccess;
        for (int i = 0; i < n_owned; ++i) {
            const hipError_t e = hipFreeAsync(owned[i], stream);
            if (first == hipSuccess) first = e;
        }
        n_owned = 0;
        if (outgrown != nullptr) {
            // an outgrown buffer no capture used: freed once the stream's work (this
            // call's launches included) is done
            hipError_t e = hipStreamSynchronize(stream);
            if (e == hipSuccess) e = hipFree(outgrown);
            outgrown = nullptr;
            if (first == hipSuccess) first = e;
        }
        return first;
    }

    char* outgrown = nullptr;  // the stream's previous buffer, freed by release()
};

// fp32 -> bf16 bits, round to nearest even (NaN kept quiet), and back.
uint16_t host_bf16(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu) != 0) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
float host_f32(uint16_t b) {
    const uint32_t u = (uint32_t)b << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// Restores the caller's current device on scope exit.
struct DeviceGuard {
    int saved = -1;
    bool changed = false;
    hipError_t enter(int device) {
        hipError_t e = hipGetDevice(&saved);
        if (e != hipSuccess) return e;
        if (saved != device) {
            e = hipSetDevice(device);
            changed = (e == hipSuccess);
        }
        return e;
    }
    ~DeviceGuard() {
        if (changed) (void)hipSetDevice(saved);
    }
};

}  // namespace

struct Gemma4QLinear {
    uint64_t magic = 0;
    Gemma4QLinearDesc desc{};  // out_features is F for a gate|up pair
    q4::Layout layout;
    int pair_rows = 0;  // F for a gate|up pair (tiled as q4::pair_layout), else 0
    const uint16_t* gelu_table = nullptr;  // the device's gelu table (pairs only)
    int device = 0;
    uint4* tiles = nullptr;  // the weight records (one allocation)
    uint2* sb = nullptr;     // their scale/bias words: kRecSbBytes into the same allocation
};

struct Gemma4QLora {
    uint64_t magic = 0;
    uint32_t rank = 0, in_features = 0, out_features = 0;
    float scale = 1.0f;
    int device = 0;
    float* a = nullptr;  // [rank, K] fp32
    float* b = nullptr;  // [N, rank] fp32
    uint16_t* a_hi = nullptr;  // A as bf16 high and low parts [ceil(rank / 16) * 16, K], rows past rank zero
    uint16_t* a_lo = nullptr;
};

namespace {

// Tiled layout of a handle: a 4-bit projection over K, an 8-bit one as two 4-bit
// planes over 2K; a gate|up pair interleaves its two projections 8 rows at a time.
q4::Layout handle_layout(const Gemma4QLinearDesc& d, bool pair) {
    const int k = (int)d.in_features * (d.bits == 8 ? 2 : 1);
    q4::Layout l = pair ? q4::pair_layout((int)d.out_features, k) : q4::make_layout((int)d.out_features, k);
    l.kx = (int)d.in_features;  // two-plane handles read x [M, K] as [x | x]
    return l;
}

Gemma4Status check_desc(const Gemma4QLinearDesc* desc, bool pair, const char* fn) {
    if (desc == nullptr) return fail(GEMMA4_ERR_INVALID_ARGUMENT, std::string(fn) + " requires a non-null desc");
    if (desc->out_features == 0 || desc->in_features == 0)
        return fail(GEMMA4_ERR_INVALID_ARGUMENT, std::string(fn) + ": out_features and in_features must be > 0");
    if ((desc->bits != 4 && desc->bits != 8) || desc->group_size != 64)
        return fail(GEMMA4_ERR_UNSUPPORTED_CONFIG,
                    std::string(fn) + ": only affine bits=4 or 8 with group_size=64 is supported (got bits=" +
                        std::to_string(desc->bits) + " group_size=" + std::to_string(desc->group_size) + ")");
    if (desc->in_features % 64 != 0)
        return fail(GEMMA4_ERR_INVALID_ARGUMENT, std::string(fn) + ": in_features must be a multiple of 64");
    if (desc->out_features > (1u << 29) || desc->in_features > (1u << 23))
        return fail(GEMMA4_ERR_UNSUPPORTED_CONFIG, std::string(fn) + ": shape exceeds the supported range");
    const q4::Layout l = handle_layout(*desc, pair);
    if (l.rec_bytes() > q4::kMaxBufferBytes)
        return fail(GEMMA4_ERR_UNSUPPORTED_CONFIG,
                    std::string(fn) + ": weights exceed 2 GiB per projection (split it along out_features)");
    return GEMMA4_OK;
}

void release(Gemma4QLinear* h) {
    if (h->tiles) (void)hipFree(h->tiles);
    h->tiles = nullptr;
    h->sb = nullptr;
    h->magic = 0;
}

bool valid_handle(const Gemma4QLinear* h) { return h != nullptr && h->magic == kQLinearMagic; }

// The layout the GEMM plans with: the handle's, without the pre-pass forms (fp16,
// one-pass 8-bit) when the process pins the bf16 form.
q4::Layout gemm_layout(const Gemma4QLinear* h) {
    q4::Layout l = h->layout;
    if (g_gemm_form.load(std::memory_order_relaxed) != 0) l.prepass_forms = false;
    return l;
}

// Whether the handle's scales allow the GEMM's fp16 form (their exponent range, from
// the device, once): sets h->layout.f16 and f16_p.
hipError_t scale_form(Gemma4QLinear* h, hipStream_t stream) {
    int* d = nullptr;
    hipError_t e = hipMalloc(&d, 3 * sizeof(int));
    if (e != hipSuccess) return e;
    const int init[3] = {-1, 255, 0};
    int range[3] = {0, 0, 1};
    e = hipMemcpyAsync(d, init, sizeof(init), hipMemcpyHostToDevice, stream);
    if (e == hipSuccess) e = q4::launch_scale_range(h->sb, h->layout, d, stream);
    if (e == hipSuccess) e = hipMemcpyAsync(range, d, sizeof(range), hipMemcpyDeviceToHost, stream);
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    (void)hipFree(d);
    if (e == hipSuccess) q4::set_f16_form(h->layout, range);
    return e;
}

// One weight triple in MLX layout (device pointers).
struct Triple {
    const uint32_t* w;
    const uint16_t* s;
    const uint16_t* b;
};

// Allocates the tiled buffers and repacks from MLX-layout device arrays: one
// projection (up == nullptr) or a gate|up pair.
Gemma4Status build_handle(const Gemma4QLinearDesc* desc, const Triple& main, const Triple* up, hipStream_t stream,
                          Gemma4QLinear** out) {
    Gemma4QLinear* h = new (std::nothrow) Gemma4QLinear();
    if (h == nullptr) return fail(GEMMA4_ERR_MEMORY_GUARD, "gemma4_qlinear: host allocation failed");
    h->desc = *desc;
    h->pair_rows = up ? (int)desc->out_features : 0;
    h->layout = handle_layout(*desc, up != nullptr);
    hipError_t e = hipGetDevice(&h->device);
    if (e != hipSuccess) {
        delete h;
        return hip_fail("hipGetDevice", e);
    }
    {
        // the device's scratch pool exists before any forward: a call under graph
        // capture may need it, and a pool cannot be created while a stream captures
        hipMemPool_t pool = nullptr;
        e = scratch_pool(h->device, &pool);
        if (e != hipSuccess) {
            delete h;
            return hip_fail("gemma4_qlinear: scratch pool", e);
        }
    }
    if (up != nullptr) {
        e = gelu_table(h->device, &h->gelu_table);
        if (e != hipSuccess) {
            delete h;
            return hip_fail("gemma4_qgeglu: gelu table", e);
        }
    }
    e = hipMalloc(&h->tiles, h->layout.rec_bytes());
    if (e == hipSuccess) h->sb = reinterpret_cast<uint2*>(reinterpret_cast<char*>(h->tiles) + q4::kRecSbBytes);
    if (e != hipSuccess) {
        release(h);
        delete h;
        return fail(GEMMA4_ERR_MEMORY_GUARD, std::string("gemma4_qlinear: device allocation failed: ") +
                                                 hipGetErrorString(e));
    }
    if (desc->bits == 8)
        e = q4::launch_repack8(main.w, main.s, main.b, up ? up->w : nullptr, up ? up->s : nullptr,
                               up ? up->b : nullptr, h->tiles, h->sb, h->layout, h->pair_rows, stream);
    else
        e = q4::launch_repack(main.w, main.s, main.b, up ? up->w : nullptr, up ? up->s : nullptr,
                              up ? up->b : nullptr, h->tiles, h->sb, h->layout, h->pair_rows, stream);
    if (e != hipSuccess) {
        release(h);
        delete h;
        return hip_fail("repack launch", e);
    }
    e = scale_form(h, stream);
    if (e != hipSuccess) {
        release(h);
        delete h;
        return hip_fail("scale range", e);
    }
    h->magic = kQLinearMagic;
    *out = h;
    return ok();
}

// Host triples -> one staging allocation -> build_handle on the null stream.
Gemma4Status create_from_host(const Gemma4QLinearDesc* desc, const uint32_t* const* w, const uint16_t* const* s,
                              const uint16_t* const* b, int parts, const char* fn, Gemma4QLinear** out) {
    const size_t n = desc->out_features, k = desc->in_features;
    const size_t wbytes = n * k * desc->bits / 8, sbytes = n * (k / 64) * 2, part = wbytes + 2 * sbytes;
    void* staging = nullptr;
    hipError_t e = hipMalloc(&staging, part * parts);
    if (e != hipSuccess)
        return fail(GEMMA4_ERR_MEMORY_GUARD, std::string(fn) + ": staging allocation failed: " + hipGetErrorString(e));
    Triple t[2];
    for (int i = 0; i < parts && e == hipSuccess; ++i) {
        char* base = static_cast<char*>(staging) + part * i;
        e = hipMemcpy(base, w[i], wbytes, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(base + wbytes, s[i], sbytes, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(base + wbytes + sbytes, b[i], sbytes, hipMemcpyHostToDevice);
        t[i] = Triple{reinterpret_cast<const uint32_t*>(base), reinterpret_cast<const uint16_t*>(base + wbytes),
                      reinterpret_cast<const uint16_t*>(base + wbytes + sbytes)};
    }
    if (e != hipSuccess) {
        (void)hipFree(staging);
        return hip_fail((std::string(fn) + ": upload").c_str(), e);
    }
    Gemma4Status st = build_handle(desc, t[0], parts == 2 ? &t[1] : nullptr, nullptr, out);
    e = hipStreamSynchronize(nullptr);
    (void)hipFree(staging);
    if (st == GEMMA4_OK && e != hipSuccess) {
        gemma4_qlinear_free(*out);
        *out = nullptr;
        return hip_fail((std::string(fn) + ": repack").c_str(), e);
    }
    return st;
}

Gemma4Status create_from_device(const Gemma4QLinearDesc* desc, const Triple& main, const Triple* up, void* stream,
                                const char* fn, Gemma4QLinear** out) {
    hipStream_t st_h = static_cast<hipStream_t>(stream);
    Gemma4Status st = build_handle(desc, main, up, st_h, out);
    if (st != GEMMA4_OK) return st;
    const hipError_t e = hipStreamSynchronize(st_h);
    if (e != hipSuccess) {
        gemma4_qlinear_free(*out);
        *out = nullptr;
        return hip_fail((std::string(fn) + ": repack").c_str(), e);
    }
    return ok();
}

// Launches one forward (checked arguments, device current) with its scratch from sc.
// With an adapter (`lora`) whose delta the GEMM's epilogue can add (an unsplit plan,
// rank a multiple of 4 up to 32), x . A^T is launched first and the GEMM adds the delta
// (*lora_done set); otherwise the caller adds it after.
Gemma4Status dispatch_forward(const Gemma4QLinear* linear, const uint16_t* x_dev, uint32_t rows, void* y_dev,
                              Gemma4QmmDtype y_dtype, bool geglu, Scratch& sc, const std::string& name,
                              const Gemma4QLora* lora = nullptr, bool* lora_done = nullptr) {
    const bool f32 = y_dtype == GEMMA4_QMM_F32;
    const int mode = geglu ? (f32 ? q4::kOutGegluF32 : q4::kOutGegluBf16) : (f32 ? q4::kOutF32 : q4::kOutBf16);
    const int n_out = linear->pair_rows;
    hipError_t e;
    if (q4::use_decode(rows, linear->layout, (int)g_gemm_min_rows.load(std::memory_order_relaxed))) {
        const q4::OutParams op{y_dev, nullptr, mode, n_out, 0, 0.0f};
        e = q4::launch_decode(linear->tiles, linear->sb, x_dev, op, (int)rows, linear->layout, sc.stream);
        if (e != hipSuccess) return hip_fail((name + ": decode launch").c_str(), e);
        return GEMMA4_OK;
    }
    // group sums of x (256-row tiles) and split-K partial sums: the unconstrained plan's
    // workspace from the pool, or what the static scratch has left (the plan then takes
    // only tiles and splits that fit that room; an unsplit plan of 64- or 128-row tiles
    // needs none)
    const q4::Layout gl = gemm_layout(linear);
    size_t ws_bytes = q4::gemm_workspace_bytes((int)rows, gl);
    if (sc.fixed) {
        ws_bytes = sc.room();
        // holds by construction (the plan takes only what fits the room); kept so that
        // a plan change can never overrun the array
        const q4::GemmPlan plan = q4::plan_gemm((int)rows, gl, ws_bytes);
        if (plan.total() > ws_bytes)
            return fail(GEMMA4_ERR_UNSUPPORTED_CONFIG, name + ": the GEMM's scratch needs more than the " +
                                                           std::to_string(kStaticScratchBytes) +
                                                           "-byte static scratch has left");
    }
    void* ws = nullptr;
    e = sc.take(sc.fixed ? 0 : ws_bytes, &ws);
    if (sc.fixed) ws = sc.base + sc.used;
    if (e != hipSuccess)
        return fail(GEMMA4_ERR_MEMORY_GUARD, name + ": workspace allocation failed: " + hipGetErrorString(e));
    q4::LoraEpilogue lo{};
    const bool with_lora = lora != nullptr && !geglu && !sc.fixed &&
                           q4::gemm_lora_epilogue((int)rows, gl, (int)lora->rank, ws_bytes);
    if (with_lora) {
        const int slices = q4::lora_slices((int)linear->desc.in_features, (int)rows);
        void* part = nullptr;
        e = sc.take((size_t)slices * rows * lora->rank * 4, &part);
        if (e != hipSuccess)
            return fail(GEMMA4_ERR_MEMORY_GUARD, name + ": workspace allocation failed: " + hipGetErrorString(e));
        e = q4::launch_lora_down(x_dev, lora->a_hi, lora->a_lo, static_cast<float*>(part), (int)rows,
                                 (int)linear->desc.in_features, (int)lora->rank, sc.stream);
        if (e != hipSuccess) return hip_fail((name + ": lora_down launch").c_str(), e);
        lo = q4::LoraEpilogue{static_cast<const float*>(part), lora->b, (int)lora->rank, slices, lora->scale};
    }
    e = q4::launch_gemm(linear->tiles, linear->sb, x_dev, y_dev, (int)rows, mode, n_out, gl, ws, ws_bytes,
                        linear->gelu_table, sc.stream, with_lora ? &lo : nullptr);
    if (e != hipSuccess) return hip_fail((name + ": gemm launch").c_str(), e);
    if (lora_done != nullptr) *lora_done = with_lora;
    return GEMMA4_OK;
}

// Checks and dispatch shared by the plain, the GeGLU and the allocation-free forward.
Gemma4Status run_forward(const Gemma4QLinear* linear, void* stream, const uint16_t* x_dev, uint32_t rows,
                         void* y_dev, Gemma4QmmDtype y_dtype, bool geglu, bool no_alloc, const char* fn,
                         const Gemma4QLora* lora = nullptr, bool* lora_done = nullptr) {
    const std::string name(fn);
    if (!valid_handle(linear)) return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + " received an invalid handle");
    if (geglu && linear->pair_rows == 0)
        return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + ": the handle is one projection, not a gate|up pair "
                                                        "(create it with gemma4_qgeglu_create)");
    if (!geglu && linear->pair_rows != 0)
        return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + ": the handle is a gate|up pair (use gemma4_qgeglu_forward)");
    if (y_dtype != GEMMA4_QMM_BF16 && y_dtype != GEMMA4_QMM_F32)
        return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + ": the output dtype must be BF16 or F32");
    if (rows == 0) return ok();
    if (x_dev == nullptr || y_dev == nullptr) return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + " requires non-null x and y");
    if ((reinterpret_cast<uintptr_t>(x_dev) & 15u) != 0)
        return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + ": x must be 16-byte aligned");
    const uintptr_t yalign = y_dtype == GEMMA4_QMM_F32 ? 3u : 1u;
    if ((reinterpret_cast<uintptr_t>(y_dev) & yalign) != 0)
        return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + ": the output is misaligned for its dtype");
    if (rows > (1u << 24)) return fail(GEMMA4_ERR_UNSUPPORTED_CONFIG, name + ": rows exceeds 2^24");
    if ((size_t)rows * linear->layout.kx * 2 > q4::kMaxBufferBytes)
        return fail(GEMMA4_ERR_UNSUPPORTED_CONFIG, name + ": x exceeds 2 GiB (split the rows into several calls)");
    DeviceGuard guard;
    hipError_t e = guard.enter(linear->device);
    if (e != hipSuccess) return hip_fail((name + ": hipSetDevice").c_str(), e);
    Scratch sc;
    sc.stream = static_cast<hipStream_t>(stream);
    sc.device = linear->device;
    if (no_alloc) {
        e = static_scratch(linear->device, &sc.base);
        if (e != hipSuccess) return hip_fail((name + ": static scratch address").c_str(), e);
        sc.fixed = true;
        sc.cap = kStaticScratchBytes;
    }
    const Gemma4Status st = dispatch_forward(linear, x_dev, rows, y_dev, y_dtype, geglu, sc, name, lora, lora_done);
    const hipError_t er = sc.release();
    if (st != GEMMA4_OK) return st;
    if (er != hipSuccess) return hip_fail((name + ": workspace release").c_str(), er);
    return ok();
}

}  // namespace

extern "C" {

Gemma4Status gemma4_qmm_runtime_version(Gemma4QmmVersionInfo* out) {
    try {
        if (out == nullptr)
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, "gemma4_qmm_runtime_version requires a non-null out pointer");
        out->abi_version = GEMMA4_QMM_ABI_VERSION;
        out->backend_name = "gemma4_qmm";
        out->backend_version = "gfx950-hip-affine-q4";
        return ok();
    } catch (...) {
        return fail_nothrow(GEMMA4_ERR_RUNTIME, "gemma4_qmm_runtime_version: unexpected native exception");
    }
}

Gemma4Status gemma4_qmm_get_last_error(char* buffer, size_t buffer_len) {
    try {
        if (buffer == nullptr || buffer_len == 0)
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, "gemma4_qmm_get_last_error requires a writable buffer");
        std::snprintf(buffer, buffer_len, "%s", g_last_error);
        return GEMMA4_OK;
    } catch (...) {
        return fail_nothrow(GEMMA4_ERR_RUNTIME, "gemma4_qmm_get_last_error: unexpected native exception");
    }
}

uint32_t gemma4_qmm_set_gemm_min_rows(uint32_t rows) {
    return g_gemm_min_rows.exchange(rows > (uint32_t)INT_MAX ? (uint32_t)INT_MAX : rows);
}

Gemma4Status gemma4_qmm_release_scratch(void* stream) {
    try {
        int device = 0;
        hipError_t e = hipGetDevice(&device);
        if (e != hipSuccess) return hip_fail("gemma4_qmm_release_scratch: hipGetDevice", e);
        const hipStream_t st = static_cast<hipStream_t>(stream);
        const std::thread::id thread = st == hipStreamPerThread ? std::this_thread::get_id() : std::thread::id();
        StreamWorkspace* ws = nullptr;
        {
            std::lock_guard<std::mutex> lock(g_ws_mu);
            for (auto& w : g_ws)
                if (w->device == device && w->stream == st && w->thread == thread) ws = w.get();
        }
        if (ws == nullptr) return ok();
        // the entry itself stays (a call in another thread may hold it); its memory goes
        std::lock_guard<std::mutex> lock(ws->mu);
        e = hipStreamSynchronize(st);
        if (e != hipSuccess) return hip_fail("gemma4_qmm_release_scratch: hipStreamSynchronize", e);
        hipError_t first = hipSuccess;
        for (char* p : ws->retired) {
            const hipError_t ef = hipFree(p);
            if (first == hipSuccess) first = ef;
        }
        ws->retired.clear();
        if (ws->buf != nullptr) {
            const hipError_t ef = hipFree(ws->buf);
            if (first == hipSuccess) first = ef;
        }
        ws->buf = nullptr;
        ws->cap = 0;
        ws->buf_captured = false;
        if (first != hipSuccess) return hip_fail("gemma4_qmm_release_scratch: hipFree", first);
        return ok();
    } catch (...) {
        return fail_nothrow(GEMMA4_ERR_RUNTIME, "gemma4_qmm_release_scratch: unexpected native exception");
    }
}

uint32_t gemma4_qmm_set_decode_kernel(uint32_t variant) {
    return (uint32_t)q4::set_decode_variant(variant > 2u ? 0 : (int)variant);
}

uint32_t gemma4_qmm_set_gemm_form(uint32_t form) { return g_gemm_form.exchange(form > 1u ? 0u : form); }

Gemma4Status gemma4_qlinear_create(const Gemma4QLinearDesc* desc, const uint32_t* weight,
                                   const uint16_t* scales, const uint16_t* biases, Gemma4QLinear** out) {
    try {
        if (out == nullptr) return fail(GEMMA4_ERR_INVALID_ARGUMENT, "gemma4_qlinear_create requires a non-null out pointer");
        *out = nullptr;
        Gemma4Status st = check_desc(desc, false, "gemma4_qlinear_create");
        if (st != GEMMA4_OK) return st;
        if (weight == nullptr || scales == nullptr || biases == nullptr)
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, "gemma4_qlinear_create requires non-null weight, scales and biases");
        return create_from_host(desc, &weight, &scales, &biases, 1, "gemma4_qlinear_create", out);
    } catch (...) {
        return fail_nothrow(GEMMA4_ERR_RUNTIME, "gemma4_qlinear_create: unexpected native exception");
    }
}

Gemma4Status gemma4_qlinear_create_device(const Gemma4QLinearDesc* desc, const uint32_t* weight_dev,
                                          const uint16_t* scales_dev, const uint16_t* biases_dev, void* stream,
                                          Gemma4QLinear** out) {
    try {
        if (out == nullptr)
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, "gemma4_qlinear_create_device requires a non-null out pointer");
        *out = nullptr;
        Gemma4Status st = check_desc(desc, false, "gemma4_qlinear_create_device");
        if (st != GEMMA4_OK) return st;
        if (weight_dev == nullptr || scales_dev == nullptr || biases_dev == nullptr)
            return fail(GEMMA4_ERR_INVALID_ARGUMENT,
                        "gemma4_qlinear_create_device requires non-null weight, scales and biases");
        return create_from_device(desc, Triple{weight_dev, scales_dev, biases_dev}, nullptr, stream,
                                  "gemma4_qlinear_create_device", out);
    } catch (...) {
        return fail_nothrow(GEMMA4_ERR_RUNTIME, "gemma4_qlinear_create_device: unexpected native exception");
    }
}

Gemma4Status gemma4_qgeglu_create(const Gemma4QLinearDesc* desc, const uint32_t* gate_weight,
                                  const uint16_t* gate_scales, const uint16_t* gate_biases, const uint32_t* up_weight,
                                  const uint16_t* up_scales, const uint16_t* up_biases, Gemma4QLinear** out) {
    try {
        if (out == nullptr) return fail(GEMMA4_ERR_INVALID_ARGUMENT, "gemma4_qgeglu_create requires a non-null out pointer");
        *out = nullptr;
        Gemma4Status st = check_desc(desc, true, "gemma4_qgeglu_create");
        if (st != GEMMA4_OK) return st;
        if (!gate_weight || !gate_scales || !gate_biases || !up_weight || !up_scales || !up_biases)
            return fail(GEMMA4_ERR_INVALID_ARGUMENT,
                        "gemma4_qgeglu_create requires non-null weight, scales and biases for gate and up");
        const uint32_t* w[2] = {gate_weight, up_weight};
        const uint16_t* s[2] = {gate_scales, up_scales};
        const uint16_t* b[2] = {gate_biases, up_biases};
        return create_from_host(desc, w, s, b, 2, "gemma4_qgeglu_create", out);
    } catch (...) {
        return fail_nothrow(GEMMA4_ERR_RUNTIME, "gemma4_qgeglu_create: unexpected native exception");
    }
}

Gemma4Status gemma4_qgeglu_create_device(const Gemma4QLinearDesc* desc, const uint32_t* gate_weight_dev,
                                         const uint16_t* gate_scales_dev, const uint16_t* gate_biases_dev,
                                         const uint32_t* up_weight_dev, const uint16_t* up_scales_dev,
                                         const uint16_t* up_biases_dev, void* stream, Gemma4QLinear** out) {
    try {
        if (out == nullptr)
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, "gemma4_qgeglu_create_device requires a non-null out pointer");
        *out = nullptr;
        Gemma4Status st = check_desc(desc, true, "gemma4_qgeglu_create_device");
        if (st != GEMMA4_OK) return st;
        if (!gate_weight_dev || !gate_scales_dev || !gate_biases_dev || !up_weight_dev || !up_scales_dev ||
            !up_biases_dev)
            return fail(GEMMA4_ERR_INVALID_ARGUMENT,
                        "gemma4_qgeglu_create_device requires non-null weight, scales and biases for gate and up");
        const Triple up{up_weight_dev, up_scales_dev, up_biases_dev};
        return create_from_device(desc, Triple{gate_weight_dev, gate_scales_dev, gate_biases_dev}, &up, stream,
                                  "gemma4_qgeglu_create_device", out);
    } catch (...) {
        return fail_nothrow(GEMMA4_ERR_RUNTIME, "gemma4_qgeglu_create_device: unexpected native exception");
    }
}

Gemma4Status gemma4_qlinear_free(Gemma4QLinear* linear) {
    try {
        if (linear == nullptr) return ok();
        if (!valid_handle(linear))
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, "gemma4_qlinear_free received an invalid handle");
        DeviceGuard guard;
        (void)guard.enter(linear->device);
        release(linear);
        delete linear;
        return ok();
    } catch (...) {
        return fail_nothrow(GEMMA4_ERR_RUNTIME, "gemma4_qlinear_free: unexpected native exception");
    }
}

Gemma4Status gemma4_qlinear_info(const Gemma4QLinear* linear, Gemma4QLinearInfo* out) {
    try {
        if (out == nullptr) return fail(GEMMA4_ERR_INVALID_ARGUMENT, "gemma4_qlinear_info requires a non-null out pointer");
        if (!valid_handle(linear))
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, "gemma4_qlinear_info received an invalid handle");
        std::memset(out, 0, sizeof(*out));
        out->out_features = linear->desc.out_features;
        out->in_features = linear->desc.in_features;
        out->bits = linear->desc.bits;
        out->group_size = linear->desc.group_size;
        out->device_bytes = linear->layout.rec_bytes();
        out->device = linear->device;
        out->flags = linear->pair_rows ? GEMMA4_QLINEAR_GEGLU_PAIR : 0u;
        return ok();
    } catch (...) {
        return fail_nothrow(GEMMA4_ERR_RUNTIME, "gemma4_qlinear_info: unexpected native exception");
    }
}

Gemma4Status gemma4_qmlp_forward(const Gemma4QLinear* gate_up, const Gemma4QLinear* down, void* stream,
                                 const uint16_t* x_dev, uint32_t rows, uint16_t* h_dev, void* y_dev,
                                 Gemma4QmmDtype y_dtype) {
    try {
        const std::string name("gemma4_qmlp_forward");
        if (!valid_handle(gate_up) || !valid_handle(down))
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + " received an invalid handle");
        if (gate_up->pair_rows == 0)
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + ": the first handle must be a gate|up pair "
                                                            "(gemma4_qgeglu_create)");
        if (down->pair_rows != 0)
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + ": the second handle must be one projection (down_proj)");
        if (down->desc.in_features != (uint32_t)gate_up->pair_rows)
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + ": down's in_features (" +
                                                         std::to_string(down->desc.in_features) +
                                                         ") must equal the pair's F (" +
                                                         std::to_string(gate_up->pair_rows) + ")");
        if (down->device != gate_up->device)
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + ": the two handles live on different devices");
        if (y_dtype != GEMMA4_QMM_BF16)
            return fail(GEMMA4_ERR_UNSUPPORTED_CONFIG, name + ": the MLP block runs in the bf16 model dtype "
                                                              "(h is bf16; under the float32 override call "
                                                              "gemma4_qgeglu_forward and gemma4_qlinear_forward)");
        if (rows == 0) return ok();
        if (x_dev == nullptr || h_dev == nullptr || y_dev == nullptr)
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + " requires non-null x, h and y");
        if ((reinterpret_cast<uintptr_t>(h_dev) & 15u) != 0)
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + ": h must be 16-byte aligned (it is down's x)");
        // the pair's launch, then down's: the two separate calls' kernels
        const Gemma4Status st = run_forward(gate_up, stream, x_dev, rows, h_dev, GEMMA4_QMM_BF16, true, false,
                                            "gemma4_qmlp_forward (gate|up)");
        if (st != GEMMA4_OK) return st;
        return run_forward(down, stream, h_dev, rows, y_dev, y_dtype, false, false, "gemma4_qmlp_forward (down)");
    } catch (...) {
        return fail_nothrow(GEMMA4_ERR_RUNTIME, "gemma4_qmlp_forward: unexpected native exception");
    }
}

Gemma4Status gemma4_qlinear_scratch_bytes(const Gemma4QLinear* linear, uint32_t rows, uint64_t* out) {
    try {
        if (out == nullptr)
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, "gemma4_qlinear_scratch_bytes requires a non-null out pointer");
        if (!valid_handle(linear))
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, "gemma4_qlinear_scratch_bytes received an invalid handle");
        *out = 0;
        if (rows == 0 || q4::use_decode(rows, linear->layout, (int)g_gemm_min_rows.load(std::memory_order_relaxed)))
            return ok();
        *out = q4::gemm_workspace_bytes((int)rows, gemm_layout(linear));
        return ok();
    } catch (...) {
        return fail_nothrow(GEMMA4_ERR_RUNTIME, "gemma4_qlinear_scratch_bytes: unexpected native exception");
    }
}

Gemma4Status gemma4_qlinear_forward(const Gemma4QLinear* linear, void* stream, const uint16_t* x_dev,
                                    uint32_t rows, void* y_dev, Gemma4QmmDtype y_dtype) {
    try {
        return run_forward(linear, stream, x_dev, rows, y_dev, y_dtype, false, false, "gemma4_qlinear_forward");
    } catch (...) {
        return fail_nothrow(GEMMA4_ERR_RUNTIME, "gemma4_qlinear_forward: unexpected native exception");
    }
}

Gemma4Status gemma4_qgeglu_forward(const Gemma4QLinear* pair, void* stream, const uint16_t* x_dev, uint32_t rows,
                                   void* h_dev, Gemma4QmmDtype h_dtype) {
    try {
        return run_forward(pair, stream, x_dev, rows, h_dev, h_dtype, true, false, "gemma4_qgeglu_forward");
    } catch (...) {
        return fail_nothrow(GEMMA4_ERR_RUNTIME, "gemma4_qgeglu_forward: unexpected native exception");
    }
}

Gemma4Status gemma4_qlinear_forward_noalloc(const Gemma4QLinear* linear, void* stream, const uint16_t* x_dev,
                                            uint32_t rows, void* y_dev, Gemma4QmmDtype y_dtype) {
    try {
        return run_forward(linear, stream, x_dev, rows, y_dev, y_dtype, false, true, "gemma4_qlinear_forward_noalloc");
    } catch (...) {
        return fail_nothrow(GEMMA4_ERR_RUNTIME, "gemma4_qlinear_forward_noalloc: unexpected native exception");
    }
}

Gemma4Status gemma4_qlinear_forward_greedy(const Gemma4QLinear* linear, void* stream, const uint16_t* x_dev,
                                           uint32_t rows, float softcap, void* logits_dev, Gemma4QmmDtype dtype,
                                           int32_t* token_dev, float* value_dev) {
    try {
        const std::string name("gemma4_qlinear_forward_greedy");
        if (!valid_handle(linear)) return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + " received an invalid handle");
        if (linear->pair_rows != 0)
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + ": the handle is a gate|up pair, not a projection");
        if (dtype != GEMMA4_QMM_BF16 && dtype != GEMMA4_QMM_F32)
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + ": dtype must be BF16 or F32");
        if (!(softcap >= 0.0f) || softcap > 3.0e38f)
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + ": softcap must be finite and >= 0 (0: none)");
        if (rows == 0) return ok();
        if (rows > (uint32_t)kGreedyMaxRows)
            return fail(GEMMA4_ERR_UNSUPPORTED_CONFIG,
                        name + ": at most " + std::to_string(kGreedyMaxRows) +
                            " rows per call (the verify block cap, gemma4_mlx.h:77-79)");
        if (x_dev == nullptr || token_dev == nullptr)
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + " requires non-null x and token outputs");
        if ((reinterpret_cast<uintptr_t>(x_dev) & 15u) != 0)
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + ": x must be 16-byte aligned");
        const uintptr_t lalign = dtype == GEMMA4_QMM_F32 ? 3u : 1u;
        if ((reinterpret_cast<uintptr_t>(logits_dev) & lalign) != 0 || (reinterpret_cast<uintptr_t>(token_dev) & 3u) != 0 ||
            (reinterpret_cast<uintptr_t>(value_dev) & 3u) != 0)
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + ": an output is misaligned for its type");
        DeviceGuard guard;
        hipError_t e = guard.enter(linear->device);
        if (e != hipSuccess) return hip_fail((name + ": hipSetDevice").c_str(), e);
        Scratch sc;
        sc.stream = static_cast<hipStream_t>(stream);
        sc.device = linear->device;
        const int nb = linear->layout.nb;
        void* part = nullptr;
        e = sc.take((size_t)rows * nb * sizeof(unsigned long long), &part);
        if (e != hipSuccess)
            return fail(GEMMA4_ERR_MEMORY_GUARD, name + ": workspace allocation failed: " + hipGetErrorString(e));
        const int mode = dtype == GEMMA4_QMM_F32 ? q4::kOutGreedyF32 : q4::kOutGreedyBf16;
        const q4::OutParams op{logits_dev, static_cast<unsigned long long*>(part), mode, 0, nb, softcap};
        Gemma4Status pst = GEMMA4_OK;
        e = q4::launch_decode(linear->tiles, linear->sb, x_dev, op, (int)rows, linear->layout, sc.stream);
        if (e == hipSuccess)
            e = q4::launch_greedy_reduce(static_cast<const unsigned long long*>(part), nb, (int)rows, token_dev,
                                         value_dev, sc.stream);
        if (e != hipSuccess) pst = hip_fail((name + ": launch").c_str(), e);
        const hipError_t ef = sc.release();
        if (pst != GEMMA4_OK) return pst;
        if (ef != hipSuccess) return hip_fail((name + ": workspace release").c_str(), ef);
        return ok();
    } catch (...) {
        return fail_nothrow(GEMMA4_ERR_RUNTIME, "gemma4_qlinear_forward_greedy: unexpected native exception");
    }
}

Gemma4Status gemma4_qlora_create(const float* a, const float* b, uint32_t rank, uint32_t in_features,
                                 uint32_t out_features, float scale, Gemma4QLora** out) {
    try {
        const std::string name("gemma4_qlora_create");
        if (out == nullptr) return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + " requires a non-null out pointer");
        *out = nullptr;
        if (a == nullptr || b == nullptr) return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + " requires non-null A and B");
        if (rank == 0 || rank > 1024 || in_features == 0 || out_features == 0 || in_features > (1u << 24) ||
            out_features > (1u << 29))
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + ": rank must be 1..1024 and the shape non-empty");
        if (!(scale == scale) || scale > 3.0e38f || scale < -3.0e38f)
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + ": scale must be finite");
        Gemma4QLora* h = new (std::nothrow) Gemma4QLora();
        if (h == nullptr) return fail(GEMMA4_ERR_MEMORY_GUARD, name + ": host allocation failed");
        h->rank = rank;
        h->in_features = in_features;
        h->out_features = out_features;
        h->scale = scale;
        hipError_t e = hipGetDevice(&h->device);
        const size_t abytes = (size_t)rank * in_features * 4, bbytes = (size_t)out_features * rank * 4;
        // A as bf16 high and low parts for the matrix-core x . A^T (rank padded to 16)
        const size_t rpad = ((size_t)rank + 15) / 16 * 16;
        std::vector<uint16_t> hi(rpad * in_features, 0), lo(rpad * in_features, 0);
        for (size_t i = 0; i < (size_t)rank * in_features; ++i) {
            hi[i] = host_bf16(a[i]);
            lo[i] = host_bf16(a[i] - host_f32(hi[i]));
        }
        const size_t sbytes = rpad * in_features * 2;
        if (e == hipSuccess) e = hipMalloc(&h->a, abytes);
        if (e == hipSuccess) e = hipMalloc(&h->b, bbytes);
        if (e == hipSuccess) e = hipMalloc(&h->a_hi, sbytes);
        if (e == hipSuccess) e = hipMalloc(&h->a_lo, sbytes);
        if (e == hipSuccess) e = hipMemcpy(h->a, a, abytes, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(h->b, b, bbytes, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(h->a_hi, hi.data(), sbytes, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(h->a_lo, lo.data(), sbytes, hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            for (void* p : {(void*)h->a, (void*)h->b, (void*)h->a_hi, (void*)h->a_lo})
                if (p) (void)hipFree(p);
            delete h;
            return fail(GEMMA4_ERR_ADAPTER, name + ": device copy failed: " + hipGetErrorString(e));
        }
        h->magic = kLoraMagic;
        *out = h;
        return ok();
    } catch (...) {
        return fail_nothrow(GEMMA4_ERR_RUNTIME, "gemma4_qlora_create: unexpected native exception");
    }
}

Gemma4Status gemma4_qlora_free(Gemma4QLora* lora) {
    try {
        if (lora == nullptr) return ok();
        if (lora->magic != kLoraMagic)
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, "gemma4_qlora_free received an invalid handle");
        DeviceGuard guard;
        (void)guard.enter(lora->device);
        (void)hipFree(lora->a);
        (void)hipFree(lora->b);
        (void)hipFree(lora->a_hi);
        (void)hipFree(lora->a_lo);
        lora->magic = 0;
        delete lora;
        return ok();
    } catch (...) {
        return fail_nothrow(GEMMA4_ERR_RUNTIME, "gemma4_qlora_free: unexpected native exception");
    }
}

Gemma4Status gemma4_qlinear_forward_lora(const Gemma4QLinear* linear, const Gemma4QLora* lora, void* stream,
                                         const uint16_t* x_dev, uint32_t rows, void* y_dev, Gemma4QmmDtype y_dtype) {
    try {
        const std::string name("gemma4_qlinear_forward_lora");
        if (lora != nullptr) {
            if (lora->magic != kLoraMagic)
                return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + " received an invalid adapter handle");
            if (valid_handle(linear) &&
                (lora->in_features != linear->desc.in_features || lora->out_features != linear->desc.out_features))
                return fail(GEMMA4_ERR_ADAPTER, name + ": adapter shape does not match the projection");
            if (valid_handle(linear) && lora->device != linear->device)
                return fail(GEMMA4_ERR_ADAPTER, name + ": adapter and projection are on different devices");
        }
        // the GEMM adds the delta in its epilogue where it can (unsplit plans, rank a
        // multiple of 4 up to 32); otherwise the LoRA kernels add it after the forward
        bool done = false;
        Gemma4Status st = run_forward(linear, stream, x_dev, rows, y_dev, y_dtype, false, false, name.c_str(), lora,
                                      &done);
        if (st != GEMMA4_OK || lora == nullptr || rows == 0 || done) return st;
        DeviceGuard guard;
        hipError_t e = guard.enter(linear->device);
        if (e != hipSuccess) return hip_fail((name + ": hipSetDevice").c_str(), e);
        Scratch sc;
        sc.stream = static_cast<hipStream_t>(stream);
        sc.device = linear->device;
        // the fused small-M launch needs no scratch
        const bool fused = q4::lora_fused((int)rows, (int)lora->rank);
        void* t = nullptr;
        if (!fused) {
            const size_t t_bytes =
                (size_t)q4::lora_slices((int)linear->desc.in_features, (int)rows) * rows * lora->rank * 4;
            e = sc.take(t_bytes, &t);
            if (e != hipSuccess)
                return fail(GEMMA4_ERR_MEMORY_GUARD, name + ": workspace allocation failed: " + hipGetErrorString(e));
        }
        e = q4::launch_lora(x_dev, lora->a, lora->a_hi, lora->a_lo, lora->b, static_cast<float*>(t), y_dev, (int)rows,
                            (int)linear->desc.out_features, (int)linear->desc.in_features, (int)lora->rank, lora->scale,
                            y_dtype == GEMMA4_QMM_F32, sc.stream);
        const hipError_t ef = sc.release();
        if (e != hipSuccess) return hip_fail((name + ": launch").c_str(), e);
        if (ef != hipSuccess) return hip_fail((name + ": workspace release").c_str(), ef);
        return ok();
    } catch (...) {
        return fail_nothrow(GEMMA4_ERR_RUNTIME, "gemma4_qlinear_forward_lora: unexpected native exception");
    }
}

Gemma4Status gemma4_qlinear_embed(const Gemma4QLinear* linear, void* stream, const int32_t* ids_dev, uint32_t count,
                                  void* out_dev, Gemma4QmmDtype dtype) {
    try {
        const std::string name("gemma4_qlinear_embed");
        if (!valid_handle(linear)) return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + " received an invalid handle");
        if (linear->pair_rows != 0)
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + ": the handle is a gate|up pair, not a projection");
        if (dtype != GEMMA4_QMM_BF16 && dtype != GEMMA4_QMM_F32)
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + ": dtype must be BF16 or F32");
        if (count == 0) return ok();
        if (ids_dev == nullptr || out_dev == nullptr)
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + " requires non-null ids and output");
        if ((reinterpret_cast<uintptr_t>(out_dev) & 15u) != 0 || (reinterpret_cast<uintptr_t>(ids_dev) & 3u) != 0)
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, name + ": ids must be 4-byte and the output 16-byte aligned");
        if (count > (1u << 24)) return fail(GEMMA4_ERR_UNSUPPORTED_CONFIG, name + ": count exceeds 2^24");
        DeviceGuard guard;
        hipError_t e = guard.enter(linear->device);
        if (e != hipSuccess) return hip_fail((name + ": hipSetDevice").c_str(), e);
        if (linear->desc.bits == 8)
            e = q4::launch_embed8(linear->tiles, linear->sb, ids_dev, (int)count, out_dev, dtype == GEMMA4_QMM_F32,
                                  linear->layout, static_cast<hipStream_t>(stream));
        else
            e = q4::launch_embed(linear->tiles, linear->sb, ids_dev, (int)count, out_dev, dtype == GEMMA4_QMM_F32,
                                 linear->layout, static_cast<hipStream_t>(stream));
        if (e != hipSuccess) return hip_fail((name + ": launch").c_str(), e);
        return ok();
    } catch (...) {
        return fail_nothrow(GEMMA4_ERR_RUNTIME, "gemma4_qlinear_embed: unexpected native exception");
    }
}

Gemma4Status gemma4_qlinear_dequantize(const Gemma4QLinear* linear, void* stream, float* w_dev) {
    try {
        if (!valid_handle(linear))
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, "gemma4_qlinear_dequantize received an invalid handle");
        if (w_dev == nullptr) return fail(GEMMA4_ERR_INVALID_ARGUMENT, "gemma4_qlinear_dequantize requires a non-null output");
        if ((reinterpret_cast<uintptr_t>(w_dev) & 15u) != 0)
            return fail(GEMMA4_ERR_INVALID_ARGUMENT, "gemma4_qlinear_dequantize: output must be 16-byte aligned");
        DeviceGuard guard;
        hipError_t e = guard.enter(linear->device);
        if (e != hipSuccess) return hip_fail("gemma4_qlinear_dequantize: hipSetDevice", e);
        if (linear->desc.bits == 8)
            e = q4::launch_dequantize8(linear->tiles, linear->sb, w_dev, linear->layout, linear->pair_rows,
                                       static_cast<hipStream_t>(stream));
        else
            e = q4::launch_dequantize(linear->tiles, linear->sb, w_dev, linear->layout, linear->pair_rows,
                                      static_cast<hipStream_t>(stream));
        if (e != hipSuccess) return hip_fail("gemma4_qlinear_dequantize: launch", e);
        return ok();
    } catch (...) {
        return fail_nothrow(GEMMA4_ERR_RUNTIME, "gemma4_qlinear_dequantize: unexpected native exception");
    }
}

}  // extern "C"
