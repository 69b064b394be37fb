// Library-wide C entry points: version, per-device init, thread-local error reporting.
// Replaces the generated host glue of the reference (src/tl_templates/tpu/main_template.cpp:14-125:
// init(), tilelang_tpu_run(), post()) with a fixed ABI; see include/tlmi355x.h.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "tlm_common.h"

static thread_local char g_last_error[512] = "";

void tlm_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int tlm_hip_fail(hipError_t e, const char* what) {
  tlm_set_error("HIP error %d (%s) in %s", (int)e, hipGetErrorString(e), what);
  return TLM_EHIP;
}

int tlm_mla_scratch_setup(int dev);  // tlm_mla.hip

namespace {
constexpr int kMaxDevices = 64;
std::once_flag g_dev_once[kMaxDevices];
int g_dev_status[kMaxDevices];
int g_dev_cus[kMaxDevices];
}  // namespace

extern "C" int tlm_version(void) { return 100; }

extern "C" const char* tlm_last_error(void) { return g_last_error; }

extern "C" int tlm_init(int device) {
  if (device < 0 || device >= kMaxDevices) {
    tlm_set_error("tlm_init: device index %d out of range", device);
    return TLM_EINVAL;
  }
  std::call_once(g_dev_once[device], [device]() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device >= n) {
      g_dev_status[device] = TLM_EHIP;
      return;
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) {
      g_dev_status[device] = TLM_EHIP;
      return;
    }
    g_dev_cus[device] = prop.multiProcessorCount;
    // The code objects are built for gfx950 only.
    if (std::string(prop.gcnArchName).rfind("gfx950", 0) != 0) {
      g_dev_status[device] = TLM_EUNSUPPORTED;
      return;
    }
    g_dev_status[device] = TLM_OK;
  });
  if (g_dev_status[device] == TLM_EHIP) {
    tlm_set_error("tlm_init: no HIP device %d", device);
    return TLM_EHIP;
  }
  if (g_dev_status[device] == TLM_EUNSUPPORTED) {
    tlm_set_error("tlm_init: device %d is not gfx950 (MI355X)", device);
    return TLM_EUNSUPPORTED;
  }
  hipError_t e = hipSetDevice(device);
  if (e != hipSuccess) return tlm_hip_fail(e, "hipSetDevice");
  // device address of the allocation-free MLA entry point's scratch array (tlm_mla.hip)
  return tlm_mla_scratch_setup(device);
}

extern "C" int tlm_num_cus(void) {
  int d = 0;
  if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= kMaxDevices) return 0;
  return g_dev_cus[d];
}
