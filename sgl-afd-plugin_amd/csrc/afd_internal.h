// Declarations shared by the translation units of libafd (not part of the C ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/afd.h"

namespace afd {

constexpr int kMaxLocalExperts = 256;
constexpr int kMaxTopk = 32;
// Widest hidden and intermediate sizes: the GEMMs gather activation rows with 32-bit offsets
// (token x row bytes, bf16 rows of up to 16384 values for up to 131071 tokens: < 2^32)
constexpr int kMaxHidden = 16384, kMaxInter = 16384;
constexpr int kBlockM = 128;  // row tile of the grouped GEMMs; expert segments pad to it
constexpr int kFp8BlockM = 256;  // the same for FP8 block weights with fp8 activations (W8A8)
// the row tile (segment padding) of a configuration's GEMMs
inline int block_m_of(const afd_moe_cfg& cfg) {
  return cfg.weight_fmt == AFD_W_FP8_BLOCK && cfg.act_fmt == AFD_A_FP8 ? kFp8BlockM : kBlockM;
}
constexpr int kMaxBatch = AFD_MAX_BATCH;  // jobs of one batched call


// Where a launch finds its job: the fields by value, or (desc != nullptr) read from the job
// descriptor in device memory when the kernel runs, its n then clamped to [0, n], n being
// here the n_cap the grids and the workspace were sized for. A batch (batch > 1) is one call
// over several jobs: job b holds the call's tokens [first[b], first[b + 1]) and its rows are
// read and written through bx[b], bids[b], bw[b] and bout[b]; n is the total.
struct JobIn {
  const afd_job* desc;
  const uint16_t* x;
  const int32_t* ids;
  const float* w;
  uint16_t* out;
  int64_t n;
  int32_t batch;
  int32_t first[kMaxBatch + 1];
  const uint16_t* bx[kMaxBatch];
  const int32_t* bids[kMaxBatch];
  const float* bw[kMaxBatch];
  uint16_t* bout[kMaxBatch];
};

// Row `t` of a batch's per-job arrays `ptrs` (rows of row_elems elements; `unit` = 1 for
// token rows, k for the flat pair index of ids / w). The selects are unrolled, so every index
// into the tables is a constant and they stay in scalar registers.
template <typename T>
__device__ __forceinline__ T* batch_row(const JobIn& j, T* const (&ptrs)[kMaxBatch], int64_t t,
                                        int64_t row_elems, int unit = 1) {
  T* p = ptrs[0];
  int64_t base = 0;
#pragma unroll
  for (int b = 1; b < kMaxBatch; ++b)
    if (b < j.batch && t >= int64_t(j.first[b]) * unit) {
      p = ptrs[b];
      base = int64_t(j.first[b]) * unit;
    }
  return p + (t - base) * row_elems;
}
// token t's x row, its out row, and the id / weight of flat pair i (= t * k + kk)
__device__ __forceinline__ const uint16_t* job_x_row(const JobIn& j, int64_t t, int cols) {
  return j.batch > 1 ? batch_row(j, j.bx, t, cols) : j.x + t * cols;
}
__device__ __forceinline__ uint16_t* job_out_row(const JobIn& j, int64_t t, int cols) {
  return j.batch > 1 ? batch_row(j, j.bout, t, cols) : j.out + t * cols;
}
__device__ __forceinline__ int32_t job_id(const JobIn& j, int64_t i, int k) {
  return j.batch > 1 ? *batch_row(j, j.bids, i, 1, k) : j.ids[i];
}
__device__ __forceinline__ const float* job_w_row(const JobIn& j, int64_t t, int k) {
  return j.batch > 1 ? batch_row(j, j.bw, t, k) : j.w + t * k;
}

__device__ __forceinline__ JobIn resolve_job(JobIn j) {
  if (j.desc != nullptr) {
    const afd_job d = *j.desc;
    j.x = d.x;
    j.ids = d.ids;
    j.w = d.w;
    j.out = d.out;
    j.n = d.n < 0 ? 0 : d.n < j.n ? d.n : j.n;
  }
  return j;
}

// Counter words of one call, in the workspace's num_tiles slot (num_tiles is word 0). Returning
// atomics on one cache line serialize (~10 ns each), so the counters that many workgroups hit
// at once each have a 256-byte line of their own: line l (l < kCounterLines) starts at word
// kLineWord0 + l * kLineStride and holds, in its words 0 / 1 / 2, the reply's group counter l,
// the gate_up GEMM's tile counter of XCD l and the down GEMM's (l < 8). The routing launch
// zeroes those words and kArriveWord before any later launch of the call uses them.
constexpr int kArriveWord = 32;  // the reply's arrive counter (one count per group)
constexpr int kLineWord0 = 64, kLineStride = 64, kCounterLines = 32;
constexpr int kArriveGroups = kCounterLines, kArriveGroupWord0 = kLineWord0, kArriveGroupStride = kLineStride;
constexpr int kGateUpWalkWord = kLineWord0 + 1;  // TileWalk: XCD x's counter x * kWalkCounterStride later
constexpr int kDownWalkWord = kLineWord0 + 2;
static_assert(kWalkCounterStride == kLineStride, "one line per XCD's tile counter");
constexpr int kCallCounterBytes = (kLineWord0 + kCounterLines * kLineStride) * 4;
inline uint32_t* call_counters(uint8_t* ws, const afd_ws_layout& L) {
  return reinterpret_cast<uint32_t*>(ws + L.num_tiles);
}

// The reply an expert call can carry (afd_moe_ffn_answer, afd_moe_ffn_batch): once every
// output row of the call is visible device-wide, *done[b] := value[b] for b < count (null
// counters skipped), stored by the last workgroup of the finalize launch to finish. arrive
// counts the finished workgroups. count == 0: no reply.
struct Reply {
  uint64_t* done[kMaxBatch];
  uint64_t value[kMaxBatch];
  int32_t count;
  uint32_t* arrive;  // kArriveWord of the call's counters; the group counters follow it
};

// Activation quantization as the expert call applies it (MXFP8 with stage-order scales, or
// FP8 1x128, by cfg.weight_fmt) into q / s.
int launch_quant_act(const afd_moe_cfg& cfg, const uint16_t* x, int32_t n, uint8_t* q, void* s,
                     hipStream_t stream);

// Routing of the job's pairs into the workspace; with quantize, the activation quantization
// of job.x into ws.xq / ws.xs (MXFP8 in stage order, or FP8 1x128, by cfg.weight_fmt) runs
// beside the expert histogram (without, the rows are quantized already). `mid` (optional)
// is recorded between the two launches.
// The first launch also zeroes the call's counter words.
int launch_route_quant(const JobIn& job, bool quantize, const afd_moe_cfg& cfg, uint8_t* ws,
                       const afd_ws_layout& L, hipStream_t stream, hipEvent_t mid);

// Grouped MXFP4 GEMMs (afd_gemm_mx.hip).
// xq / xs: the quantized activation rows [n][H] and their scales (the workspace's, or the
// caller's for afd_moe_ffn_q); with rows_desc != nullptr they are read from that job
// descriptor's xq / xs when the kernel runs.
int launch_mx_gate_up(const afd_moe_cfg& cfg, const afd_expert_weights& wt, uint8_t* ws,
                      const afd_ws_layout& L, const uint8_t* xq, const void* xs,
                      const afd_job* rows_desc, hipStream_t stream);
int launch_mx_down(const afd_moe_cfg& cfg, const afd_expert_weights& wt, uint8_t* ws,
                   const afd_ws_layout& L, int32_t n, hipStream_t stream);

// Grouped MXFP4-weight x bf16-activation GEMMs (afd_gemm_a16.hip). x: the bf16 token rows
// [n][H] (the job's, or a batch's staged in the workspace); with rows_desc != nullptr they are
// that job descriptor's x, read when the kernel runs.
int launch_a16_gate_up(const afd_moe_cfg& cfg, const afd_expert_weights& wt, uint8_t* ws,
                       const afd_ws_layout& L, const uint16_t* x, const afd_job* rows_desc,
                       hipStream_t stream);
int launch_a16_down(const afd_moe_cfg& cfg, const afd_expert_weights& wt, uint8_t* ws,
                    const afd_ws_layout& L, hipStream_t stream);

// Grouped FP8 128x128-block GEMMs (afd_gemm_fp8.hip).
int launch_fp8_gate_up(const afd_moe_cfg& cfg, const afd_expert_weights& wt, uint8_t* ws,
                       const afd_ws_layout& L, const uint8_t* xq, const void* xs,
                       const afd_job* rows_desc, hipStream_t stream);
int launch_fp8_down(const afd_moe_cfg& cfg, const afd_expert_weights& wt, uint8_t* ws,
                    const afd_ws_layout& L, int32_t n, hipStream_t stream);

// Number of compute units of the current device (cached per device).
int device_cu_count();

}  // namespace afd
