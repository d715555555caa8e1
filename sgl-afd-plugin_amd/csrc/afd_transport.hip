// Transport primitives of the one-GPU A<->F loop: pinned host flag pages, device copies and
// 64-bit stream memops. The memops run on the stream's own queue, so a producer stream rings
// a doorbell and a consumer stream parks on it without any host thread waiting.
#include <cstring>

#include "afd_common.h"
#include "afd_internal.h"

extern "C" int afd_host_alloc(void** ptr, uint64_t bytes) {
  if (!ptr || bytes == 0) return AFD_ERR_ARG;
  *ptr = nullptr;
  AFD_CHECK_HIP(hipHostMalloc(ptr, bytes, hipHostMallocCoherent | hipHostMallocPortable));
  std::memset(*ptr, 0, bytes);
  return AFD_OK;
}

extern "C" int afd_host_free(void* ptr) {
  if (!ptr) return AFD_OK;
  AFD_CHECK_HIP(hipHostFree(ptr));
  return AFD_OK;
}

extern "C" int afd_copy_async(void* dst, const void* src, uint64_t bytes, afd_stream_t stream) {
  if (bytes == 0) return AFD_OK;
  if (!dst || !src) return AFD_ERR_ARG;
  AFD_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice,
                               static_cast<hipStream_t>(stream)));
  return AFD_OK;
}

extern "C" int afd_stream_write64(afd_stream_t stream, uint64_t* addr, uint64_t value) {
  if (!addr || (reinterpret_cast<uintptr_t>(addr) & 7)) return AFD_ERR_ARG;
  AFD_CHECK_HIP(hipStreamWriteValue64(static_cast<hipStream_t>(stream), addr, value, 0));
  return AFD_OK;
}

extern "C" int afd_stream_wait64(afd_stream_t stream, uint64_t* addr, uint64_t value,
                                 uint64_t mask, int32_t cond) {
  if (!addr || (reinterpret_cast<uintptr_t>(addr) & 7)) return AFD_ERR_ARG;
  unsigned flags;
  switch (cond) {
    case AFD_WAIT_GEQ: flags = hipStreamWaitValueGte; break;
    case AFD_WAIT_EQ: flags = hipStreamWaitValueEq; break;
    case AFD_WAIT_AND: flags = hipStreamWaitValueAnd; break;
    case AFD_WAIT_NOR: flags = hipStreamWaitValueNor; break;
    default: return AFD_ERR_ARG;
  }
  AFD_CHECK_HIP(
      hipStreamWaitValue64(static_cast<hipStream_t>(stream), addr, value, flags, mask));
  return AFD_OK;
}
