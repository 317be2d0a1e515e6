// runtime.hip - contexts, device memory, copies and the error convention of libh3hip.so (the HIP counterpart of
// kernels/h3sycl.cpp:77-402), and the entry points of kernels/h3sycl.h that have no implementation here.
#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <tuple>

#include "common.h"

namespace h3 {

thread_local std::string g_err;
static std::atomic<uint64_t> g_allocs{0};
void count_alloc() { g_allocs.fetch_add(1, std::memory_order_relaxed); }
void set_error(const std::string& msg) { g_err = msg; }
int fail(const std::string& msg) { g_err = msg; return -1; }

Ctx* ctx_of(void* ctx, const char* fn) {
    if (!ctx) { set_error(std::string(fn) + ": no context"); return nullptr; }
    Ctx* c = static_cast<Ctx*>(ctx);
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess || cur != c->device) (void) hipSetDevice(c->device);
    return c;
}

int blocks_per_cu(const void* kernel, int threads, size_t lds) {
    static std::mutex mu;
    static std::map<std::tuple<const void*, int, size_t>, int> known;
    std::lock_guard<std::mutex> l(mu);
    const auto key = std::make_tuple(kernel, threads, lds);
    const auto it = known.find(key);
    if (it != known.end()) return it->second;
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, lds) != hipSuccess || n < 1) {
        (void) hipGetLastError();
        n = 1;
    }
    known.emplace(key, n);
    return n;
}

int launched(const char* fn) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(std::string(fn) + ": kernel launch failed: " + hipGetErrorString(e));
    return 0;
}

PhaseTimer::PhaseTimer(Ctx* c, bool allowed) : c_(c), on_(allowed && c->profile) {}
PhaseTimer::~PhaseTimer() {
    for (hipEvent_t e : ev_) (void) hipEventDestroy(e);
}
void PhaseTimer::mark() {
    if (!on_) return;
    hipEvent_t e = nullptr;
    count_alloc();
    if (hipEventCreate(&e) != hipSuccess) { on_ = false; (void) hipGetLastError(); return; }
    ev_.push_back(e);
    (void) hipEventRecord(e, c_->stream);
}
std::vector<float> PhaseTimer::elapsed() {
    std::vector<float> out;
    if (!on_ || ev_.size() < 2) return out;
    (void) hipEventSynchronize(ev_.back());
    for (size_t i = 1; i < ev_.size(); ++i) {
        float ms = 0.0f;
        (void) hipEventElapsedTime(&ms, ev_[i - 1], ev_[i]);
        out.push_back(ms);
    }
    return out;
}

static std::string mib(size_t bytes) { return std::to_string((bytes + (1 << 20) - 1) >> 20) + " MiB"; }

bool Budget::take(size_t bytes, const std::string& what) {
    std::lock_guard<std::mutex> l(mu_);
    if (in_use_ <= limit_ && bytes <= limit_ - in_use_) {
        in_use_ += bytes;
        return true;
    }
    set_error(what + ": " + mib(bytes) + " more would exceed this context's device memory budget (" + mib(in_use_) +
              " of " + mib(limit_) + " taken; H3S_MEM_FRACTION sets the budget)");
    return false;
}

bool Budget::forget(void* p) {
    std::lock_guard<std::mutex> l(mu_);
    const auto it = buffers_.find(p);
    if (it == buffers_.end()) return false;
    in_use_ -= it->second < in_use_ ? it->second : in_use_;
    buffers_.erase(it);
    return true;
}

std::vector<void*> Budget::buffers() const {
    std::lock_guard<std::mutex> l(mu_);
    std::vector<void*> out;
    for (const auto& kv : buffers_) out.push_back(kv.first);
    return out;
}

static const char* region_name(Ctx::Region r) {
    switch (r) {
        case Ctx::LIN_CODES: return "int8 linear scratch (quantized rows)";
        case Ctx::LIN_SCALES: return "int8 linear scratch (row scales)";
        case Ctx::ATT_Q: return "attention scratch (q)";
        case Ctx::ATT_K: return "attention scratch (k)";
        case Ctx::ATT_V: return "attention scratch (v)";
        case Ctx::ATT_AUX: return "attention scratch (scales and k's mean)";
        case Ctx::ATT_PART: return "attention scratch (partial sums)";
        case Ctx::LIN_F32: return "linear scratch (float32 product)";
        default: return "scratch";
    }
}

// Regions grow to whole 2 MiB granules (the device's allocation granule for large buffers), so a region that needs a
// few more rows than last time is not reallocated at every call. The old region goes first, once the queued kernels
// that may use it are done, so the budget never holds both.
void* Ctx::scratch_bytes(Region r, size_t bytes) {
    constexpr size_t kGranule = (size_t) 2 << 20;
    Area& a = areas[r];
    if (bytes <= a.bytes) return a.p;
    const size_t want = (bytes + kGranule - 1) / kGranule * kGranule;
    if (a.p) {
        (void) hipStreamSynchronize(stream);
        (void) hipFree(a.p);
        budget.give_back(a.bytes);
        a = Area{};
    }
    if (!budget.take(want, region_name(r))) return nullptr;
    void* p = nullptr;
    count_alloc();
    if (hipMalloc(&p, want) != hipSuccess || !p) {
        (void) hipGetLastError();
        budget.give_back(want);
        set_error(std::string(region_name(r)) + ": hipMalloc of " + mib(want) + " failed");
        return nullptr;
    }
    if (poison) (void) hipMemsetAsync(p, 0xff, want, stream);
    a.p = p;
    a.bytes = want;
    return p;
}

// what every way of making a context shares: the device's name and the memory cap (kernels/h3sycl.cpp:216-235)
static void init(Ctx& c) {
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, c.device) == hipSuccess) {
        c.name = p.name;
        if (c.name.empty() || c.name.find("gfx") == 0) c.name = std::string(p.gcnArchName);
        if (p.multiProcessorCount > 0) c.cus = p.multiProcessorCount;
    }
    // H3S_CUS: the compute units that grids are sized by (fewer than the device's: tests of the grid shapes)
    if (const char* e = std::getenv("H3S_CUS")) c.cus = std::max(1, std::min(c.cus, std::atoi(e)));
    size_t free_b = 0, total = 0;
    (void) hipMemGetInfo(&free_b, &total);
    double frac = 0.94;
    if (const char* e = std::getenv("H3S_MEM_FRACTION")) frac = std::min(0.97, std::max(0.05, std::atof(e)));
    c.budget.set_limit((size_t) ((double) total * frac));
    c.poison = std::getenv("H3S_POISON") != nullptr;
    c.profile = std::getenv("H3S_PROFILE") != nullptr;
    // h3s_int8_linear_noalloc's fixed scratch: its address on this device, looked up once (a failure is reported by
    // that entry point, not here)
    (void) noalloc_setup(c.device);
    // the attention form (kernels/h3sycl.cpp:231-232): H3S_ATTN=onednn keeps every call on the 16-bit form;
    // H3S_SAGE_MIN_S sets the shortest sequence that takes the int8 (SageAttention) form
    if (const char* e = std::getenv("H3S_ATTN")) c.sage_want = std::strcmp(e, "onednn") != 0;
    if (const char* e = std::getenv("H3S_SAGE_MIN_S")) c.sage_min_s = std::max<int64_t>(0, std::atoll(e));
    // the pipelined attention kernel: a last round of blocks that fills at most half the CUs is split into up to this
    // many key ranges a block (1: never)
    if (const char* e = std::getenv("H3S_ATTN_SPLIT")) c.attn_split = std::max(1, std::min(64, std::atoi(e)));
    // the row quantizer's layout: one wavefront a row from this many rows on (four wavefronts a row below)
    if (const char* e = std::getenv("H3S_QUANT_WAVE_MIN_ROWS")) c.quant_wave_min = std::max<int64_t>(0, std::atoll(e));
}

static Ctx* open_on(int index) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) { set_error("no GPU"); return nullptr; }
    if (index < 0 || index >= n) { set_error("no GPU " + std::to_string(index) + " (" + std::to_string(n) + " found)"); return nullptr; }
    if (hipSetDevice(index) != hipSuccess) { set_error("hipSetDevice failed"); return nullptr; }
    auto* c = new Ctx;
    c->device = index;
    count_alloc();
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        set_error("could not create a stream");
        return nullptr;
    }
    c->own_stream = true;
    init(*c);
    return c;
}

}  // namespace h3

using namespace h3;

H3S_EXPORT const char* h3s_last_error(void) { return g_err.c_str(); }

H3S_EXPORT void* h3s_open(void) try { return open_on(0); } catch (const std::exception& e) { set_error(e.what()); return nullptr; }

H3S_EXPORT void* h3s_open_gpu(int index) try { return open_on(index); } catch (const std::exception& e) { set_error(e.what()); return nullptr; }

H3S_EXPORT void* h3s_create(void* hip_stream) try {
    auto* c = new Ctx;
    if (hipGetDevice(&c->device) != hipSuccess) { delete c; set_error("no current GPU"); return nullptr; }
    c->stream = static_cast<hipStream_t>(hip_stream);
    c->own_stream = false;
    init(*c);
    return c;
} catch (const std::exception& e) { set_error(e.what()); return nullptr; }

H3S_EXPORT int h3s_gpu_count(void) {
    int n = 0;
    const hipError_t e = hipGetDeviceCount(&n);
    if (e == hipErrorNoDevice) return 0;
    if (e != hipSuccess) return fail(std::string("hipGetDeviceCount: ") + hipGetErrorString(e));
    return n;
}

H3S_EXPORT int h3s_gpu_info(int index, char* name, int name_len, uint64_t* mem_bytes, char* pci, int pci_len) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || index < 0 || index >= n) return fail("no GPU " + std::to_string(index));
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, index) != hipSuccess) return fail("hipGetDeviceProperties failed");
    if (name && name_len > 0) std::snprintf(name, (size_t) name_len, "%s", p.name);
    if (mem_bytes) *mem_bytes = (uint64_t) p.totalGlobalMem;
    if (pci && pci_len > 0) std::snprintf(pci, (size_t) pci_len, "%04x:%02x:%02x.0", p.pciDomainID, p.pciBusID, p.pciDeviceID);
    return 0;
}

H3S_EXPORT void* h3s_stream(void* ctx) { return ctx ? static_cast<Ctx*>(ctx)->stream : nullptr; }

H3S_EXPORT const char* h3s_device_name(void* ctx) { return ctx ? static_cast<Ctx*>(ctx)->name.c_str() : ""; }

H3S_EXPORT uint64_t h3s_mem_cap(void* ctx) { return ctx ? static_cast<Ctx*>(ctx)->budget.limit() : 0; }

H3S_EXPORT uint64_t h3s_mem_used(void* ctx) { return ctx ? static_cast<Ctx*>(ctx)->budget.in_use() : 0; }

H3S_EXPORT uint64_t h3s_mem_free(void* ctx) {
    if (!ctx_of(ctx, "h3s_mem_free")) return 0;
    size_t free_b = 0, total = 0;
    return hipMemGetInfo(&free_b, &total) == hipSuccess ? free_b : 0;
}

// Device memory for the caller, counted against the context's budget. A zero-byte request still returns a distinct
// buffer (one 256-byte allocation granule), so the pointer can be freed like any other.
H3S_EXPORT void* h3s_alloc(void* ctx, uint64_t bytes) try {
    Ctx* c = ctx_of(ctx, "h3s_alloc");
    if (!c) return nullptr;
    if (!c->budget.take(bytes, "h3s_alloc")) return nullptr;
    void* p = nullptr;
    count_alloc();
    if (hipMalloc(&p, bytes ? bytes : 256) != hipSuccess || !p) {
        (void) hipGetLastError();
        c->budget.give_back(bytes);
        set_error("h3s_alloc: hipMalloc of " + mib(bytes) + " failed");
        return nullptr;
    }
    if (c->poison && hipMemset(p, 0xff, bytes ? bytes : 256) != hipSuccess) {
        (void) hipFree(p);
        c->budget.give_back(bytes);
        set_error("h3s_alloc: filling the new buffer with 0xff (H3S_POISON) failed");
        return nullptr;
    }
    c->budget.remember(p, bytes);
    return p;
} catch (const std::exception& e) { set_error(e.what()); return nullptr; }

// Frees a buffer of h3s_alloc once the work queued on the context (kernels and uploads) is done with it; any other
// pointer is left alone.
H3S_EXPORT void h3s_free(void* ctx, void* p) {
    Ctx* c = ctx_of(ctx, "h3s_free");
    if (!c || !p) return;
    (void) hipStreamSynchronize(c->stream);
    if (c->copy_stream) (void) hipStreamSynchronize(c->copy_stream);
    if (c->budget.forget(p)) (void) hipFree(p);
}

H3S_EXPORT int h3s_write(void* ctx, void* dst, const void* src_host, uint64_t bytes) {
    Ctx* c = ctx_of(ctx, "h3s_write");
    if (!c) return -1;
    if (!bytes) return 0;
    hipError_t e = hipMemcpyAsync(dst, src_host, bytes, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    return e == hipSuccess ? 0 : fail(std::string("h3s_write: ") + hipGetErrorString(e));
}

H3S_EXPORT int h3s_read(void* ctx, void* dst_host, const void* src, uint64_t bytes) {
    Ctx* c = ctx_of(ctx, "h3s_read");
    if (!c) return -1;
    if (!bytes) return 0;
    hipError_t e = hipMemcpyAsync(dst_host, src, bytes, hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    return e == hipSuccess ? 0 : fail(std::string("h3s_read: ") + hipGetErrorString(e));
}

H3S_EXPORT int h3s_copy(void* ctx, void* dst, const void* src, uint64_t bytes) {
    Ctx* c = ctx_of(ctx, "h3s_copy");
    if (!c) return -1;
    if (!bytes) return 0;
    const hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, c->stream);
    return e == hipSuccess ? 0 : fail(std::string("h3s_copy: ") + hipGetErrorString(e));
}

H3S_EXPORT int h3s_wait(void* ctx) {
    Ctx* c = ctx_of(ctx, "h3s_wait");
    if (!c) return -1;
    const hipError_t e = hipStreamSynchronize(c->stream);
    return e == hipSuccess ? 0 : fail(std::string("h3s_wait: ") + hipGetErrorString(e));
}

H3S_EXPORT void* h3s_alloc_host(void* ctx, uint64_t bytes) {
    Ctx* c = ctx_of(ctx, "h3s_alloc_host");
    if (!c) return nullptr;
    void* p = nullptr;
    count_alloc();
    if (hipHostMalloc(&p, bytes ? bytes : 1, hipHostMallocDefault) != hipSuccess) {
        set_error("h3s_alloc_host: the runtime refused " + std::to_string(bytes >> 20) + " MiB of pinned memory");
        return nullptr;
    }
    return p;
}

H3S_EXPORT void h3s_free_host(void* ctx, void* p) {
    Ctx* c = ctx_of(ctx, "h3s_free_host");
    if (!c || !p) return;
    if (c->copy_stream) (void) hipStreamSynchronize(c->copy_stream);
    (void) hipHostFree(p);
}

// Device allocations, host allocations, events, streams and library handles the library has made in this process,
// counted as they are attempted: a diagnostic that shows a call path allocates nothing.
H3S_EXPORT uint64_t h3s_alloc_count(void) { return g_allocs.load(std::memory_order_relaxed); }

H3S_EXPORT int h3s_upload(void* ctx, void* dst, const void* src_pinned, uint64_t bytes) {
    Ctx* c = ctx_of(ctx, "h3s_upload");
    if (!c) return -1;
    hipPointerAttribute_t a, b;
    if (hipPointerGetAttributes(&a, src_pinned) != hipSuccess || a.type != hipMemoryTypeHost ||
        hipPointerGetAttributes(&b, dst) != hipSuccess || b.type != hipMemoryTypeDevice) {
        (void) hipGetLastError();
        return fail("h3s_upload: the source must be h3s_alloc_host memory and the destination device memory");
    }
    {
        std::lock_guard<std::mutex> l(c->copy_mu);
        if (!c->copy_stream) count_alloc();
        if (!c->copy_stream && hipStreamCreateWithFlags(&c->copy_stream, hipStreamNonBlocking) != hipSuccess)
            return fail("h3s_upload: could not create the copy stream");
    }
    if (!bytes) return 0;
    const hipError_t e = hipMemcpyAsync(dst, src_pinned, bytes, hipMemcpyHostToDevice, c->copy_stream);
    return e == hipSuccess ? 0 : fail(std::string("h3s_upload: ") + hipGetErrorString(e));
}

H3S_EXPORT int h3s_upload_wait(void* ctx) {
    Ctx* c = ctx_of(ctx, "h3s_upload_wait");
    if (!c) return -1;
    if (!c->copy_stream) return 0;
    const hipError_t e = hipStreamSynchronize(c->copy_stream);
    return e == hipSuccess ? 0 : fail(std::string("h3s_upload_wait: ") + hipGetErrorString(e));
}

H3S_EXPORT void h3s_destroy(void* ctx) {
    if (!ctx) return;
    auto* c = static_cast<Ctx*>(ctx);
    (void) hipSetDevice(c->device);
    (void) hipStreamSynchronize(c->stream);
    if (c->copy_stream) { (void) hipStreamSynchronize(c->copy_stream); (void) hipStreamDestroy(c->copy_stream); }
    if (c->profile && c->lin_chunks)
        std::fprintf(stderr, "h3hip: int8 linear, %lld row chunks: quantize %.1f ms, int8 GEMM %.1f ms\n",
                     (long long) c->lin_chunks, c->lin_ms[0], c->lin_ms[1]);
    for (auto& a : c->areas)
        if (a.p) (void) hipFree(a.p);
    release_blas(c);
    for (void* p : c->budget.buffers()) (void) hipFree(p);
    if (c->own_stream) (void) hipStreamDestroy(c->stream);
    delete c;
}

// ---- entry points of kernels/h3sycl.h outside this library's scope: present (engine/h3-sys resolves every name,
// engine/h3-sys/src/lib.rs:233-281) and refusing, with the reason ----
#define H3S_NOT_HERE(name, what) \
    return fail(std::string(name) + ": not implemented in libh3hip (" what "); only the per-token layer kernels are")

H3S_EXPORT int h3s_dequant(void*, const void*, int, int64_t, void*, int) { H3S_NOT_HERE("h3s_dequant", "k-quant weights"); }
H3S_EXPORT int h3s_conv3d(void*, const void*, int, int64_t, int64_t, int64_t, int64_t, const void*, int64_t, int64_t, const float*, void*) {
    H3S_NOT_HERE("h3s_conv3d", "convolution");
}
H3S_EXPORT int h3s_group_norm_silu(void*, const void*, int, int64_t, int64_t, int64_t, int64_t, const float*, const float*, float,
                                   const float*, const float*, void*) {
    H3S_NOT_HERE("h3s_group_norm_silu", "upscaler");
}
H3S_EXPORT int h3s_pad3d(void*, const void*, int, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, void*) {
    H3S_NOT_HERE("h3s_pad3d", "upscaler");
}
H3S_EXPORT int h3s_conv2d(void*, const void*, int, int64_t, int64_t, int64_t, int64_t, const void*, int64_t, int64_t, const float*, void*) {
    H3S_NOT_HERE("h3s_conv2d", "convolution");
}
H3S_EXPORT int h3s_prelu(void*, void*, int, int64_t, int64_t, const float*) { H3S_NOT_HERE("h3s_prelu", "upscaler"); }
H3S_EXPORT int h3s_pixel_shuffle_add(void*, const void*, int, int64_t, int64_t, int64_t, int64_t, int64_t, const void*, void*) {
    H3S_NOT_HERE("h3s_pixel_shuffle_add", "upscaler");
}
H3S_EXPORT int h3s_resize_area(void*, const void*, int, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, float*) {
    H3S_NOT_HERE("h3s_resize_area", "upscaler");
}
H3S_EXPORT int h3s_conv3d_ex(void*, const void*, int, int64_t, int64_t, int64_t, int64_t, const void*, int64_t, int64_t, int64_t, int64_t,
                             int64_t, int64_t, int64_t, const float*, void*) {
    H3S_NOT_HERE("h3s_conv3d_ex", "convolution");
}
H3S_EXPORT int h3s_temporal_dwconv(void*, const void*, int, int64_t, int64_t, int64_t, const float*, int64_t, const float*, void*) {
    H3S_NOT_HERE("h3s_temporal_dwconv", "convolution");
}
H3S_EXPORT int h3s_trilinear(void*, const void*, int, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, void*) {
    H3S_NOT_HERE("h3s_trilinear", "upscaler");
}
H3S_EXPORT int h3s_conv1d(void*, const float*, int64_t, int64_t, int64_t, const float*, int64_t, int64_t, const float*, int64_t, int64_t,
                          int64_t, float*, int64_t) {
    H3S_NOT_HERE("h3s_conv1d", "audio");
}
H3S_EXPORT int h3s_conv_transpose1d(void*, const float*, int64_t, int64_t, int64_t, const float*, int64_t, int64_t, const float*, int64_t,
                                    int64_t, float*, int64_t) {
    H3S_NOT_HERE("h3s_conv_transpose1d", "audio");
}
H3S_EXPORT int h3s_aa_snake(void*, const float*, int64_t, int64_t, int64_t, const float*, const float*, const float*, const float*, float*) {
    H3S_NOT_HERE("h3s_aa_snake", "audio");
}
H3S_EXPORT int h3s_scale(void*, float*, int64_t, float) { H3S_NOT_HERE("h3s_scale", "audio"); }
H3S_EXPORT int h3s_snake(void*, const float*, int64_t, int64_t, int64_t, const float*, float*) { H3S_NOT_HERE("h3s_snake", "audio"); }
