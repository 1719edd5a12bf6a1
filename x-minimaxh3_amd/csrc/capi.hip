// Error reporting and host-side launch helpers shared by every C-ABI entry point of libmx_qlinear.so.
#include <stdarg.h>
#include <stdio.h>

#include "mxq_common.h"

#include <mutex>

static thread_local char g_last_error[512] = "";

int mxq_set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int mxq_check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return mxq_set_error(MXQ_ERR_HIP, "%s launch failed: %s", what, hipGetErrorString(err));
  return MXQ_OK;
}

// Compute units of the current device, cached per device (256 when the query fails).
int mxq_cu_count() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    cached[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
  }
  return cached[dev];
}

int mxq_blocks_per_cu(const void* kernel, int block, size_t lds) {
  struct Entry {
    const void* kernel;
    int dev, block;
    size_t lds;
    int per_cu;
  };
  static std::mutex mu;
  static Entry cache[64];
  static int used = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  {
    std::lock_guard<std::mutex> lock(mu);
    for (int i = 0; i < used; ++i)
      if (cache[i].kernel == kernel && cache[i].dev == dev && cache[i].block == block && cache[i].lds == lds)
        return cache[i].per_cu;
  }
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block, lds) != hipSuccess || per_cu < 1) per_cu = 1;
  std::lock_guard<std::mutex> lock(mu);
  if (used < 64) cache[used++] = Entry{kernel, dev, block, lds, per_cu};
  return per_cu;
}

extern "C" const char* mxq_last_error(void) { return g_last_error; }

extern "C" int mxq_abi_version(void) { return MXQ_ABI_VERSION; }
