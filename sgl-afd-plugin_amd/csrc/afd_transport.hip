// Transport of the one-GPU A<->F loop: pinned host flag pages, the message send (backpressure
// waits, payload copies, doorbells) and the reply (partial-sum copies, done counters) as one
// call each, and the stream memops they are made of. Everything runs on the caller's stream,
// so a producer stream rings a doorbell and a consumer stream parks on it without any host
// thread waiting.
//
// Done flags are 64-bit message counters that only grow, waited on with an unsigned >=
// compare: a wait for message s is satisfied by s and by every later message, so any store of
// a larger count (the next reply, or a watchdog's release) frees every earlier wait. Doorbell
// words keep the reference's 32-bit sequence field.
#include <cstring>

#include "afd_common.h"
#include "afd_internal.h"

namespace {

// The payload copies of a message or a reply, enqueued as hipMemcpyAsync device-to-device
// copies: measured against one fused copy kernel, they left the compute kernels of other
// streams more of the GPU (the one-GPU loop 7% and the skewed job stream 6% faster).
constexpr int kMaxCopies = 4 * AFD_MAX_F;

struct CopyList {
  int count = 0;
  const void* src[kMaxCopies];
  void* dst[kMaxCopies];
  uint64_t bytes[kMaxCopies];
  bool add(const void* s, void* d, uint64_t n) {
    if (n == 0 || s == d) return true;
    if (count == kMaxCopies) return false;
    src[count] = s;
    dst[count] = d;
    bytes[count] = n;
    ++count;
    return true;
  }
  int enqueue(hipStream_t stream) const {
    for (int i = 0; i < count; ++i)
      AFD_CHECK_HIP(hipMemcpyAsync(dst[i], src[i], bytes[i], hipMemcpyDeviceToDevice, stream));
    return AFD_OK;
  }
};

bool aligned8(const void* p) { return p != nullptr && (reinterpret_cast<uintptr_t>(p) & 7) == 0; }

}  // namespace

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
  if (!aligned8(addr)) return AFD_ERR_ARG;
  AFD_CHECK_HIP(hipStreamWriteValue64(static_cast<hipStream_t>(stream), addr, value, 0));
  return AFD_OK;
}

extern "C" int afd_stream_wait64(afd_stream_t stream, uint64_t* addr, uint64_t value,
                                 uint64_t mask, int32_t cond) {
  if (!aligned8(addr)) return AFD_ERR_ARG;
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

extern "C" int afd_send(const afd_send_desc* m, afd_stream_t stream) {
  if (!m || m->num_f < 1 || m->num_f > AFD_MAX_F) return AFD_ERR_ARG;
  if (!m->x || !m->ids || !m->w || m->x_bytes == 0 || m->ids_bytes == 0) return AFD_ERR_ARG;
  if ((m->xs == nullptr) != (m->xs_bytes == 0)) return AFD_ERR_ARG;
  // the fields must not overlap inside a region: x | xs | ids | w
  const uint64_t x_end = m->x_bytes;
  if (m->xs && (m->xs_off < x_end || m->xs_off + m->xs_bytes > m->ids_off)) return AFD_ERR_ARG;
  if (m->ids_off < x_end || m->ids_off + m->ids_bytes > m->w_off) return AFD_ERR_ARG;
  CopyList copies;
  for (int f = 0; f < m->num_f; ++f) {
    uint8_t* region = static_cast<uint8_t*>(m->region[f]);
    if (!region || !aligned8(m->bell[f])) return AFD_ERR_ARG;
    if (m->done[f] && !aligned8(m->done[f])) return AFD_ERR_ARG;
    copies.add(m->x, region, m->x_bytes);
    if (m->xs) copies.add(m->xs, region + m->xs_off, m->xs_bytes);
    copies.add(m->ids, region + m->ids_off, m->ids_bytes);
    copies.add(m->w, region + m->w_off, m->ids_bytes);  // fp32 weights: as many bytes as the ids
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  // backpressure: the previous message of this slot must be answered by every F rank before
  // its region is overwritten
  for (int f = 0; f < m->num_f; ++f)
    if (m->done[f])
      AFD_CHECK_HIP(hipStreamWaitValue64(s, m->done[f], m->done_min, hipStreamWaitValueGte,
                                         ~uint64_t(0)));
  const int rc = copies.enqueue(s);
  if (rc != AFD_OK) return rc;
  // the doorbells follow the copies on the same stream: a consumer that sees one sees the payload
  for (int f = 0; f < m->num_f; ++f)
    AFD_CHECK_HIP(hipStreamWriteValue64(s, m->bell[f], m->word[f], 0));
  return AFD_OK;
}

extern "C" int afd_reply(const afd_reply_desc* rows, int32_t num_rows, afd_stream_t stream) {
  if (!rows || num_rows < 1 || num_rows > kMaxCopies) return AFD_ERR_ARG;
  CopyList copies;
  for (int r = 0; r < num_rows; ++r) {
    if (!aligned8(rows[r].done)) return AFD_ERR_ARG;
    if (rows[r].bytes && (!rows[r].src || !rows[r].dst)) return AFD_ERR_ARG;
    copies.add(rows[r].src, rows[r].dst, rows[r].bytes);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int rc = copies.enqueue(s);
  if (rc != AFD_OK) return rc;
  for (int r = 0; r < num_rows; ++r)
    AFD_CHECK_HIP(hipStreamWriteValue64(s, rows[r].done, rows[r].value, 0));
  return AFD_OK;
}

extern "C" int afd_wait_replies(uint64_t* const* done, int32_t num_f, uint64_t seq,
                                afd_stream_t stream) {
  if (!done || num_f < 1 || num_f > AFD_MAX_F) return AFD_ERR_ARG;
  for (int f = 0; f < num_f; ++f)
    if (!aligned8(done[f])) return AFD_ERR_ARG;
  hipStream_t s = static_cast<hipStream_t>(stream);
  for (int f = 0; f < num_f; ++f)
    AFD_CHECK_HIP(hipStreamWaitValue64(s, done[f], seq, hipStreamWaitValueGte, ~uint64_t(0)));
  return AFD_OK;
}
