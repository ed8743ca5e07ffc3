#include "hip_rt.h"
#include "kargs.h"

#include <dlfcn.h>

#include <cstdio>
#include <cstring>
#include <mutex>

extern "C" const unsigned char hat_kernels_co_start[];
extern "C" const unsigned char hat_kernels_co_end[];

namespace hat {

const std::vector<std::string>& required_kernels()
{
    static const std::vector<std::string> k = {
        "hat_attn_sw_d24",     "hat_attn_sw_d30",     "hat_attn_oca_d24",   "hat_attn_oca_d30",
        "hat_attnx_sw_d24",    "hat_attnx_sw_d30",    "hat_attnx_oca_d24",  "hat_attnx_oca_d30",
        "hat_gemmx_qkv", "hat_gemmx_qkv180", "hat_mlpx180_ln", "hat_mlpx180", "hat_projx180_hab", "hat_projx180",       "hat_projx_cab",       "hat_projx",          "hat_mlpx_ln", "hat_habx_cab_ln", "hat_habx", "hat_habx180_hab_ln", "hat_habx180", "hat_attnx_swp_d30",
        "hat_mlpx", "hat_conv_first_ln144", "hat_conv_first_ln180",
        "hat_conv_n1_store",   "hat_conv_n3_store",   "hat_conv_n4_store",  "hat_conv_n3_resid",
        "hat_conv_n3_colsum",  "hat_conv_n4_shuffle", "hat_conv_n1_final", "hat_conv_last3",
        "hat_gemm_n9_store",   "hat_gemm_n9_gelu",    "hat_gemm_n9_qkv",    "hat_gemm_n9_resid",
        "hat_gemm_n9_resid_ln", "hat_gemm_n9_hab_ln",
        "hat_gemm_n12_store",  "hat_gemm_n12_gelu",   "hat_gemm_n12_qkv",   "hat_gemm_n12_resid",
        "hat_gemm_n12_resid_ln", "hat_gemm_n12_hab_ln",
        "hat_gemmws_qkv",      "hat_gemmws_gelu",     "hat_gemmws_resid_ln", "hat_gemmws_hab_ln",
        "hat_gemmws12_qkv",    "hat_gemmws12_gelu",   "hat_gemmws12_resid_ln", "hat_gemmws12_hab_ln",
        "hat_mlp_resid",       "hat_mlp_resid_ln",    "hat_mlp12_resid",    "hat_mlp12_resid_ln",    "hat_gemmws_cab_ln",  "hat_cab_conv1",  "hat_cab_conv1_t32",
        "hat_cab_gate",        "hat_convw_n9_store_ln", "hat_convw_n9_resid_ln", "hat_convwino_resid", "hat_convwino_n4_store", "hat_convwino_n8_shuffle", "hat_convwino_resid180", "hat_convwino_n4_store180",
        "hat_convwino_cab1_180", "hat_convwino_cab2_180", "hat_convw_n9_resid",
        "hat_convw_n4_store",  "hat_convw_n8_shuffle", "hat_convw_n6_resid", "hat_convw_n6_colsum", "hat_hab_tail", "hat_ocab_tail",
        "hat_layernorm",       "hat_pre",             "hat_colsum_reduce",  "hat_se_gate",
        "hat_copy",
    };
    return k;
}

namespace {

void* open_hip(std::string* why)
{
    const char* names[] = {"libamdhip64.so.7", "libamdhip64.so", "/opt/rocm/lib/libamdhip64.so"};
    for (const char* n : names) {
        void* h = dlopen(n, RTLD_NOW | RTLD_LOCAL);
        if (h) return h;
    }
    if (why) *why = std::string("cannot dlopen libamdhip64: ") + (dlerror() ? dlerror() : "?");
    return nullptr;
}

template <class F>
void sym(void* lib, F& f, const char* name)
{
    void* p = dlsym(lib, name);
    if (!p) throw Error(std::string("libamdhip64 has no `") + name + "`");
    f = reinterpret_cast<F>(p);
}

}  // namespace

bool gpu_available(std::string* why)
{
    void* lib = open_hip(why);
    if (!lib) return false;
    hipError_t (*init)(unsigned) = nullptr;
    hipError_t (*count)(int*) = nullptr;
    init = reinterpret_cast<hipError_t (*)(unsigned)>(dlsym(lib, "hipInit"));
    count = reinterpret_cast<hipError_t (*)(int*)>(dlsym(lib, "hipGetDeviceCount"));
    if (!init || !count) {
        if (why) *why = "libamdhip64 lacks hipInit/hipGetDeviceCount";
        return false;
    }
    if (init(0) != hipSuccess) {
        if (why) *why = "hipInit failed: no usable GPU driver";
        return false;
    }
    int n = 0;
    if (count(&n) != hipSuccess || n < 1) {
        if (why) *why = "no HIP device";
        return false;
    }
    return true;
}

Runtime& Runtime::get()
{
    static std::mutex mu;
    static Runtime* rt = nullptr;
    std::lock_guard<std::mutex> g(mu);
    if (!rt) rt = new Runtime();  // lives until the process ends
    return *rt;
}

Runtime::Runtime()
{
    std::string why;
    api_.lib = open_hip(&why);
    if (!api_.lib) throw Error(why);
    void* l = api_.lib;
    sym(l, api_.Init, "hipInit");
    sym(l, api_.GetDeviceCount, "hipGetDeviceCount");
    sym(l, api_.SetDevice, "hipSetDevice");
    sym(l, api_.DeviceSynchronize, "hipDeviceSynchronize");
    sym(l, api_.GetErrorString, "hipGetErrorString");
    sym(l, api_.DeviceGetName, "hipDeviceGetName");
    sym(l, api_.DeviceGetAttribute, "hipDeviceGetAttribute");
    sym(l, api_.ModuleLoadData, "hipModuleLoadData");
    sym(l, api_.ModuleUnload, "hipModuleUnload");
    sym(l, api_.ModuleGetFunction, "hipModuleGetFunction");
    sym(l, api_.ModuleGetGlobal, "hipModuleGetGlobal");
    sym(l, api_.ModuleLaunchKernel, "hipModuleLaunchKernel");
    sym(l, api_.Malloc, "hipMalloc");
    sym(l, api_.Free, "hipFree");
    sym(l, api_.Memcpy, "hipMemcpy");
    sym(l, api_.MemcpyAsync, "hipMemcpyAsync");
    sym(l, api_.Memcpy2DAsync, "hipMemcpy2DAsync");
    sym(l, api_.MemGetInfo, "hipMemGetInfo");
    sym(l, api_.HostMalloc, "hipHostMalloc");
    sym(l, api_.HostFree, "hipHostFree");
    sym(l, api_.StreamCreate, "hipStreamCreate");
    sym(l, api_.StreamDestroy, "hipStreamDestroy");
    sym(l, api_.StreamSynchronize, "hipStreamSynchronize");
    sym(l, api_.EventCreate, "hipEventCreate");
    sym(l, api_.EventCreateWithFlags, "hipEventCreateWithFlags");
    sym(l, api_.EventDestroy, "hipEventDestroy");
    sym(l, api_.EventRecord, "hipEventRecord");
    sym(l, api_.StreamWaitEvent, "hipStreamWaitEvent");
    sym(l, api_.EventSynchronize, "hipEventSynchronize");
    sym(l, api_.EventElapsedTime, "hipEventElapsedTime");

    check(api_.Init(0), "hipInit");
    int n = 0;
    check(api_.GetDeviceCount(&n), "hipGetDeviceCount");
    if (n < 1) throw Error("no HIP device");
    check(api_.SetDevice(0), "hipSetDevice(0)");
    check(api_.ModuleLoadData(&module_, hat_kernels_co_start), "hipModuleLoadData(gfx950 kernels)");
    for (const std::string& k : required_kernels()) {
        hipFunction_t f = nullptr;
        hipError_t e = api_.ModuleGetFunction(&f, module_, k.c_str());
        if (e != hipSuccess || !f)
            throw Error("the embedded code object has no kernel `" + k +
                        "`: the kernel list and the sources disagree");
        fns_[k] = f;
        names_.push_back(k);
    }
    // The device address of the scratch array, resolved once with device 0
    // current. The kernels live in a module loaded at run time, so host code
    // has no symbol for the array at all: this pointer is the only handle.
    hipDeviceptr_t sp = nullptr;
    size_t sb = 0;
    check(api_.ModuleGetGlobal(&sp, &sb, module_, "hat_scratch"), "hipModuleGetGlobal(hat_scratch)");
    if (!sp || sb != (size_t)hatk::SCRATCH_BYTES)
        throw Error("the code object's scratch array is " + std::to_string(sb) + " bytes, expected " +
                    std::to_string((size_t)hatk::SCRATCH_BYTES));
    scratch_ = sp;
    scratch_bytes_ = sb;
}

void Runtime::check(hipError_t e, const char* what) const
{
    if (e != hipSuccess) {
        const char* s = api_.GetErrorString ? api_.GetErrorString(e) : "?";
        throw Error(std::string(what) + ": " + s + " (" + std::to_string((int)e) + ")");
    }
}

hipFunction_t Runtime::fn(const char* name) const
{
    auto it = fns_.find(name);
    if (it == fns_.end()) throw Error(std::string("unknown kernel `") + name + "`");
    return it->second;
}

std::string Runtime::device_name() const
{
    char buf[256] = {0};
    if (api_.DeviceGetName(buf, sizeof buf, 0) != hipSuccess) return "?";
    // Some boards report no marketing name; the code object only loads on
    // gfx950, so that is what the device is.
    if (buf[0] == '\0') return "gfx950";
    return buf;
}

int Runtime::cu_count() const
{
    int v = 0;
    api_.DeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, 0);
    return v;
}

void* Runtime::alloc(size_t bytes)
{
    void* p = nullptr;
    if (bytes == 0) bytes = 4;
    hipError_t e = api_.Malloc(&p, bytes);
    if (e != hipSuccess) {
        size_t fr = 0, tot = 0;
        api_.MemGetInfo(&fr, &tot);
        char b[256];
        snprintf(b, sizeof b, "hipMalloc(%.1f MiB) failed with %.1f of %.1f GiB free", bytes / 1048576.0,
                 fr / 1073741824.0, tot / 1073741824.0);
        throw Error(b);
    }
    return p;
}

void Runtime::free(void* p)
{
    if (p) api_.Free(p);
}

void Runtime::h2d(void* dst, const void* src, size_t bytes)
{
    check(api_.Memcpy(dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
}

void Runtime::d2h(void* dst, const void* src, size_t bytes)
{
    check(api_.Memcpy(dst, src, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
}

void Runtime::sync() { check(api_.DeviceSynchronize(), "hipDeviceSynchronize"); }

// ---------------------------------------------------------------------------
// Per-kernel event timing.

namespace {
struct Pending {
    std::string name;
    hipEvent_t a, b;
};
struct Profiler {
    bool on = false;
    std::vector<Pending> pending;
    std::vector<hipEvent_t> pool;
    std::vector<KernelStat> stats;
    hipEvent_t take(const HipApi& api)
    {
        if (!pool.empty()) {
            hipEvent_t e = pool.back();
            pool.pop_back();
            return e;
        }
        hipEvent_t e = nullptr;
        api.EventCreate(&e);
        return e;
    }
};
Profiler& prof()
{
    static Profiler p;
    return p;
}
}  // namespace

void profile_begin()
{
    prof().on = true;
    prof().stats.clear();
    prof().pending.clear();
}

void profile_collect()
{
    Profiler& p = prof();
    const HipApi& api = Runtime::get().api();
    for (Pending& e : p.pending) {
        api.EventSynchronize(e.b);
        float ms = 0.0f;
        api.EventElapsedTime(&ms, e.a, e.b);
        KernelStat* st = nullptr;
        for (KernelStat& s : p.stats)
            if (s.name == e.name) st = &s;
        if (!st) {
            p.stats.push_back(KernelStat{e.name, 0, 0.0});
            st = &p.stats.back();
        }
        st->count += 1;
        st->total_ms += ms;
        p.pool.push_back(e.a);
        p.pool.push_back(e.b);
    }
    p.pending.clear();
}

std::vector<KernelStat> profile_stats() { return prof().stats; }

void profile_end()
{
    profile_collect();
    prof().on = false;
}

void launch_raw(hipStream_t stream, const char* name, unsigned gx, unsigned gy, unsigned gz,
                unsigned bx, const void* args, size_t size)
{
    Runtime& rt = Runtime::get();
    const HipApi& api = rt.api();
    hipFunction_t f = rt.fn(name);
    if (gx == 0 || gy == 0 || gz == 0) return;
    // The kernarg segment holds exactly the argument struct.
    alignas(16) unsigned char buf[512];
    if (size > sizeof buf) throw Error("kernel argument block too large");
    memcpy(buf, args, size);
    size_t sz = size;
    void* cfg[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, buf, HIP_LAUNCH_PARAM_BUFFER_SIZE, &sz,
                   HIP_LAUNCH_PARAM_END};
    Profiler& p = prof();
    hipEvent_t ea = nullptr, eb = nullptr;
    if (p.on) {
        ea = p.take(api);
        eb = p.take(api);
        api.EventRecord(ea, stream);
    }
    rt.check(api.ModuleLaunchKernel(f, gx, gy, gz, bx, 1, 1, 0, stream, nullptr, cfg), name);
    if (p.on) {
        api.EventRecord(eb, stream);
        p.pending.push_back(Pending{name, ea, eb});
    }
}

}  // namespace hat
