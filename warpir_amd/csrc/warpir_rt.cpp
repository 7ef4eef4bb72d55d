// C-ABI launcher of the WarpIR MI355X backend: a thin layer over the HIP
// module API.  Declarations and conventions: include/warpir_rt.h.
#include "warpir_rt.h"

#include <hip/hip_runtime.h>

#include <cstring>

extern "C" {

int wir_abi_version(void) { return WIR_RT_ABI_VERSION; }

int wir_set_device(int device) { return (int)hipSetDevice(device); }

int wir_device_info(int device, int* num_cus, int* clock_khz, int* lds_per_block, char* arch,
                    size_t arch_len) {
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return (int)e;
  if (num_cus) *num_cus = prop.multiProcessorCount;
  if (clock_khz) *clock_khz = prop.clockRate;
  if (lds_per_block) *lds_per_block = (int)prop.sharedMemPerBlock;
  if (arch && arch_len) {
    std::strncpy(arch, prop.gcnArchName, arch_len - 1);
    arch[arch_len - 1] = '\0';
  }
  return 0;
}

int wir_module_load(const void* image, size_t size, wir_module_t* module) {
  if (!image || !size || !module) return (int)hipErrorInvalidValue;
  hipModule_t m = nullptr;
  hipError_t e = hipModuleLoadData(&m, image);
  if (e != hipSuccess) return (int)e;
  *module = (wir_module_t)m;
  return 0;
}

int wir_module_unload(wir_module_t module) {
  if (!module) return (int)hipErrorInvalidValue;
  return (int)hipModuleUnload((hipModule_t)module);
}

int wir_module_get_function(wir_module_t module, const char* name, wir_function_t* function) {
  if (!module || !name || !function) return (int)hipErrorInvalidValue;
  hipFunction_t f = nullptr;
  hipError_t e = hipModuleGetFunction(&f, (hipModule_t)module, name);
  if (e != hipSuccess) return (int)e;
  *function = (wir_function_t)f;
  return 0;
}

int wir_launch(wir_function_t function, unsigned gx, unsigned gy, unsigned gz, unsigned bx,
               unsigned by, unsigned bz, unsigned dyn_lds, void* stream, const void* kernarg,
               size_t kernarg_size) {
  if (!function || !gx || !gy || !gz || !bx || !by || !bz) return (int)hipErrorInvalidValue;
  if (kernarg_size && !kernarg) return (int)hipErrorInvalidValue;
  size_t size = kernarg_size;
  void* config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, const_cast<void*>(kernarg),
                    HIP_LAUNCH_PARAM_BUFFER_SIZE, &size, HIP_LAUNCH_PARAM_END};
  return (int)hipModuleLaunchKernel((hipFunction_t)function, gx, gy, gz, bx, by, bz, dyn_lds,
                                    (hipStream_t)stream, nullptr, config);
}

int wir_function_attrs(wir_function_t function, int* num_regs, int* static_lds, int* max_threads) {
  if (!function) return (int)hipErrorInvalidValue;
  hipFunction_t f = (hipFunction_t)function;
  hipError_t e;
  int v = 0;
  if (num_regs) {
    e = hipFuncGetAttribute(&v, HIP_FUNC_ATTRIBUTE_NUM_REGS, f);
    if (e != hipSuccess) return (int)e;
    *num_regs = v;
  }
  if (static_lds) {
    e = hipFuncGetAttribute(&v, HIP_FUNC_ATTRIBUTE_SHARED_SIZE_BYTES, f);
    if (e != hipSuccess) return (int)e;
    *static_lds = v;
  }
  if (max_threads) {
    e = hipFuncGetAttribute(&v, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, f);
    if (e != hipSuccess) return (int)e;
    *max_threads = v;
  }
  return 0;
}

int wir_stream_sync(void* stream) { return (int)hipStreamSynchronize((hipStream_t)stream); }

int wir_device_sync(void) { return (int)hipDeviceSynchronize(); }

int wir_event_create(wir_event_t* event) {
  if (!event) return (int)hipErrorInvalidValue;
  hipEvent_t ev = nullptr;
  hipError_t e = hipEventCreate(&ev);
  if (e != hipSuccess) return (int)e;
  *event = (wir_event_t)ev;
  return 0;
}

int wir_event_destroy(wir_event_t event) { return (int)hipEventDestroy((hipEvent_t)event); }

int wir_event_record(wir_event_t event, void* stream) {
  return (int)hipEventRecord((hipEvent_t)event, (hipStream_t)stream);
}

int wir_event_elapsed_ms(wir_event_t start, wir_event_t end, float* ms) {
  if (!ms) return (int)hipErrorInvalidValue;
  hipError_t e = hipEventSynchronize((hipEvent_t)end);
  if (e != hipSuccess) return (int)e;
  return (int)hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)end);
}

const char* wir_error_string(int code) {
  if (code == WIR_ERROR_SCRATCH_LIMIT)
    return "input exceeds the library's device scratch (splits * M * N > WIR_NOALLOC_SCRATCH_FLOATS)";
  return hipGetErrorString((hipError_t)code);
}

}  // extern "C"
