// runtime.hip - contexts, device memory, copies and the error convention of libh3hip.so (the HIP counterpart of
// kernels/h3sycl.cpp:77-402), and the entry points of kernels/h3sycl.h that have no implementation here.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <tuple>

#include "common.h"

namespace h3 {

thread_local std::string g_err;
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

// what every way of making a context shares: the device's name and the memory cap (kernels/h3sycl.cpp:216-235)
static void init(Ctx& c) {
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, c.device) == hipSuccess) {
        c.name = p.name;
        if (c.name.empty() || c.name.find("gfx") == 0) c.name = std::string(p.gcnArchName);
        if (p.multiProcessorCount > 0) c.cus = p.multiProcessorCount;
    }
    size_t free_b = 0, total = 0;
    (void) hipMemGetInfo(&free_b, &total);
    double frac = 0.94;
    if (const char* e = std::getenv("H3S_MEM_FRACTION")) frac = std::min(0.97, std::max(0.05, std::atof(e)));
    c.mem_cap = (size_t) ((double) total * frac);
    c.poison = std::getenv("H3S_POISON") != nullptr;
    // the attention form (kernels/h3sycl.cpp:231-232): H3S_ATTN=onednn keeps every call on the 16-bit form;
    // H3S_SAGE_MIN_S sets the shortest sequence that takes the int8 (SageAttention) form
    if (const char* e = std::getenv("H3S_ATTN")) c.sage_want = std::strcmp(e, "onednn") != 0;
    if (const char* e = std::getenv("H3S_SAGE_MIN_S")) c.sage_min_s = std::max<int64_t>(0, std::atoll(e));
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

H3S_EXPORT uint64_t h3s_mem_cap(void* ctx) { return ctx ? static_cast<Ctx*>(ctx)->mem_cap : 0; }

H3S_EXPORT uint64_t h3s_mem_used(void* ctx) {
    if (!ctx) return 0;
    auto& c = *static_cast<Ctx*>(ctx);
    std::lock_guard<std::mutex> l(c.mem_mu);
    return c.mem_used;
}

H3S_EXPORT uint64_t h3s_mem_free(void* ctx) {
    if (!ctx_of(ctx, "h3s_mem_free")) return 0;
    size_t free_b = 0, total = 0;
    return hipMemGetInfo(&free_b, &total) == hipSuccess ? free_b : 0;
}

H3S_EXPORT void* h3s_alloc(void* ctx, uint64_t bytes) try {
    Ctx* c = ctx_of(ctx, "h3s_alloc");
    if (!c) return nullptr;
    std::lock_guard<std::mutex> l(c->mem_mu);
    if (c->mem_used + bytes > c->mem_cap) {
        set_error("h3s_alloc: " + std::to_string(bytes >> 20) + " MiB would pass the device memory cap (" +
                  std::to_string(c->mem_used >> 20) + " of " + std::to_string(c->mem_cap >> 20) + " MiB in use)");
        return nullptr;
    }
    void* p = nullptr;
    if (hipMalloc(&p, bytes ? bytes : 1) != hipSuccess) {
        set_error("h3s_alloc: the device refused " + std::to_string(bytes >> 20) + " MiB");
        return nullptr;
    }
    if (c->poison && hipMemset(p, 0xff, bytes ? bytes : 1) != hipSuccess) {
        (void) hipFree(p);
        set_error("h3s_alloc: poisoning the buffer failed");
        return nullptr;
    }
    c->mem.emplace(p, bytes);
    c->mem_used += bytes;
    return p;
} catch (const std::exception& e) { set_error(e.what()); return nullptr; }

H3S_EXPORT void h3s_free(void* ctx, void* p) {
    Ctx* c = ctx_of(ctx, "h3s_free");
    if (!c || !p) return;
    (void) hipStreamSynchronize(c->stream);          // nothing queued may still read or write it
    if (c->copy_stream) (void) hipStreamSynchronize(c->copy_stream);
    std::lock_guard<std::mutex> l(c->mem_mu);
    auto it = c->mem.find(p);
    if (it == c->mem.end()) return;
    c->mem_used -= it->second;
    c->mem.erase(it);
    (void) hipFree(p);
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
    if (c->xq) (void) hipFree(c->xq);
    if (c->rs) (void) hipFree(c->rs);
    for (void* p : {(void*) c->aq, (void*) c->ak, (void*) c->av, (void*) c->af, (void*) c->lin})
        if (p) (void) hipFree(p);
    release_blas(c);
    for (auto& kv : c->mem) (void) hipFree(kv.first);
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
