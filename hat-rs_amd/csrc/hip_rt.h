// The HIP runtime, loaded at run time.
//
// The reference reaches its GPU through lightgpu::vm, which dlopens
// libcuda.so.1 and resolves the driver entry points by name (src/cuda.rs:
// 34-41, README.md:19-23). This is the MI355X counterpart: libamdhip64 is
// dlopened on first use, so the library itself has no link-time dependency on
// ROCm and loads (and answers every host-only call) on a machine without a GPU.
// The gfx950 code object is embedded in the library and loaded with
// hipModuleLoadData; every kernel is resolved by name at start-up.
#pragma once
#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

namespace hat {

struct Error {
    std::string msg;
    explicit Error(std::string m) : msg(std::move(m)) {}
};

struct HipApi {
    void* lib = nullptr;
    hipError_t (*Init)(unsigned int);
    hipError_t (*GetDeviceCount)(int*);
    hipError_t (*SetDevice)(int);
    hipError_t (*DeviceSynchronize)();
    const char* (*GetErrorString)(hipError_t);
    hipError_t (*DeviceGetName)(char*, int, int);
    hipError_t (*DeviceGetAttribute)(int*, hipDeviceAttribute_t, int);
    hipError_t (*ModuleLoadData)(hipModule_t*, const void*);
    hipError_t (*ModuleUnload)(hipModule_t);
    hipError_t (*ModuleGetFunction)(hipFunction_t*, hipModule_t, const char*);
    hipError_t (*ModuleGetGlobal)(hipDeviceptr_t*, size_t*, hipModule_t, const char*);
    hipError_t (*ModuleLaunchKernel)(hipFunction_t, unsigned, unsigned, unsigned, unsigned,
                                     unsigned, unsigned, unsigned, hipStream_t, void**, void**);
    hipError_t (*Malloc)(void**, size_t);
    hipError_t (*Free)(void*);
    hipError_t (*Memcpy)(void*, const void*, size_t, hipMemcpyKind);
    hipError_t (*MemcpyAsync)(void*, const void*, size_t, hipMemcpyKind, hipStream_t);
    hipError_t (*Memcpy2DAsync)(void*, size_t, const void*, size_t, size_t, size_t, hipMemcpyKind, hipStream_t);
    hipError_t (*MemGetInfo)(size_t*, size_t*);
    hipError_t (*HostMalloc)(void**, size_t, unsigned int);
    hipError_t (*HostFree)(void*);
    hipError_t (*StreamCreate)(hipStream_t*);
    hipError_t (*StreamDestroy)(hipStream_t);
    hipError_t (*StreamSynchronize)(hipStream_t);
    hipError_t (*StreamWaitEvent)(hipStream_t, hipEvent_t, unsigned);
    hipError_t (*EventCreate)(hipEvent_t*);
    hipError_t (*EventCreateWithFlags)(hipEvent_t*, unsigned);
    hipError_t (*EventDestroy)(hipEvent_t);
    hipError_t (*EventRecord)(hipEvent_t, hipStream_t);
    hipError_t (*EventSynchronize)(hipEvent_t);
    hipError_t (*EventElapsedTime)(float*, hipEvent_t, hipEvent_t);
};

// The process-wide runtime: the dlopened API, device 0, the loaded module and
// the kernel table. Created on first use; throws hat::Error when no driver or
// device can be brought up.
class Runtime {
public:
    static Runtime& get();
    const HipApi& api() const { return api_; }
    hipFunction_t fn(const char* name) const;
    const std::vector<std::string>& kernel_names() const { return names_; }
    std::string device_name() const;
    int cu_count() const;
    void check(hipError_t e, const char* what) const;

    void* alloc(size_t bytes);
    void free(void* p);
    void h2d(void* dst, const void* src, size_t bytes);
    void d2h(void* dst, const void* src, size_t bytes);
    void sync();
    // The code object's fixed scratch array (hat_scratch) on this device, as
    // hipModuleGetGlobal reports it at start-up; used only by forward_noalloc.
    void* scratch() const { return scratch_; }
    size_t scratch_bytes() const { return scratch_bytes_; }

private:
    Runtime();
    HipApi api_{};
    hipModule_t module_ = nullptr;
    std::unordered_map<std::string, hipFunction_t> fns_;
    std::vector<std::string> names_;
    void* scratch_ = nullptr;
    size_t scratch_bytes_ = 0;
};

// True if the HIP runtime library can be opened and reports a device. Never
// throws; used by callers that want to ask before committing.
bool gpu_available(std::string* why);

// The names of every kernel the embedded code object must provide.
const std::vector<std::string>& required_kernels();

// A launch: one argument struct copied into the kernarg segment.
template <class A>
void launch(hipStream_t stream, const char* name, unsigned gx, unsigned gy, unsigned gz,
            unsigned bx, const A& args);
void launch_raw(hipStream_t stream, const char* name, unsigned gx, unsigned gy, unsigned gz,
                unsigned bx, const void* args, size_t size);

template <class A>
inline void launch(hipStream_t stream, const char* name, unsigned gx, unsigned gy, unsigned gz,
                   unsigned bx, const A& args)
{
    launch_raw(stream, name, gx, gy, gz, bx, &args, sizeof(A));
}

// Per-kernel timing with HIP events recorded on the launch stream. While a
// recorder is active every launch is bracketed by two events; `collect` waits
// for them and accumulates the elapsed time per kernel name.
struct KernelStat {
    std::string name;
    long count = 0;
    double total_ms = 0.0;
};
void profile_begin();
void profile_collect();                       // after the stream has been synchronised
std::vector<KernelStat> profile_stats();
void profile_end();

}  // namespace hat
