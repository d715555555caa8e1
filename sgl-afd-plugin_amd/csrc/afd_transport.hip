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

// One launch copies up to kMaxCopies byte ranges: the four fields of a message to every F
// rank, or the partial sums of a job's rows. Each workgroup copies one 16 KiB piece of one
// range; the range of a workgroup is found from the prefix of piece counts (a scalar walk
// over at most kMaxCopies entries).
constexpr int kMaxCopies = 4 * AFD_MAX_F;
constexpr int kCopyThreads = 256;
constexpr int kCopyUnroll = 4;
constexpr uint64_t kPieceBytes = uint64_t(kCopyThreads) * kCopyUnroll * 16;

struct CopyPlan {
  int32_t count;
  uint32_t first_piece[kMaxCopies + 1];
  const uint8_t* src[kMaxCopies];
  uint8_t* dst[kMaxCopies];
  uint64_t bytes[kMaxCopies];
};

__global__ __launch_bounds__(kCopyThreads) void copy_plan_kernel(CopyPlan plan) {
  const uint32_t piece = blockIdx.x;
  int i = 0;
  while (i + 1 < plan.count && piece >= plan.first_piece[i + 1]) ++i;
  const uint64_t base = uint64_t(piece - plan.first_piece[i]) * kPieceBytes;
  const uint8_t* src = plan.src[i];
  uint8_t* dst = plan.dst[i];
  const uint64_t bytes = plan.bytes[i];
  const int t = threadIdx.x;
  if (((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) == 0) {
    uint4 v[kCopyUnroll];
#pragma unroll
    for (int j = 0; j < kCopyUnroll; ++j) {
      const uint64_t off = base + uint64_t(t + j * kCopyThreads) * 16;
      if (off + 16 <= bytes) v[j] = *reinterpret_cast<const uint4*>(src + off);
    }
#pragma unroll
    for (int j = 0; j < kCopyUnroll; ++j) {
      const uint64_t off = base + uint64_t(t + j * kCopyThreads) * 16;
      if (off + 16 <= bytes) *reinterpret_cast<uint4*>(dst + off) = v[j];
    }
    const uint64_t whole = bytes & ~uint64_t(15);  // the last < 16 bytes, by the piece holding them
    if (whole < bytes && whole >= base && whole < base + kPieceBytes && uint64_t(t) < bytes - whole)
      dst[whole + t] = src[whole + t];
  } else {  // a range that is not 16-byte aligned (a sliced ids / weights view): byte by byte
    for (int j = 0; j < int(kPieceBytes / kCopyThreads); ++j) {
      const uint64_t off = base + uint64_t(j) * kCopyThreads + t;
      if (off < bytes) dst[off] = src[off];
    }
  }
}

struct CopyList {
  CopyPlan plan{};
  bool add(const void* src, void* dst, uint64_t bytes) {
    if (bytes == 0 || src == dst) return true;
    if (plan.count == kMaxCopies) return false;
    plan.src[plan.count] = static_cast<const uint8_t*>(src);
    plan.dst[plan.count] = static_cast<uint8_t*>(dst);
    plan.bytes[plan.count] = bytes;
    ++plan.count;
    return true;
  }
  int enqueue(hipStream_t stream) {
    uint64_t pieces = 0;
    for (int i = 0; i < plan.count; ++i) {
      plan.first_piece[i] = static_cast<uint32_t>(pieces);
      pieces += (plan.bytes[i] + kPieceBytes - 1) / kPieceBytes;
      if (pieces >= (1ull << 31)) return AFD_ERR_ARG;
    }
    plan.first_piece[plan.count] = static_cast<uint32_t>(pieces);
    if (pieces == 0) return AFD_OK;
    hipLaunchKernelGGL(copy_plan_kernel, dim3(static_cast<uint32_t>(pieces)), dim3(kCopyThreads), 0,
                       stream, plan);
    AFD_CHECK_LAUNCH();
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
