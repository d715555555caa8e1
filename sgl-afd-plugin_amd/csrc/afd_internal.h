// Declarations shared by the translation units of libafd (not part of the C ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/afd.h"

namespace afd {

constexpr int kMaxLocalExperts = 256;
constexpr int kMaxTopk = 32;
constexpr int kBlockM = 128;  // row tile of the grouped GEMMs; expert segments pad to it


// Where a launch finds its job: the fields by value, or (desc != nullptr) read from the job
// descriptor in device memory when the kernel runs, its n then clamped to [0, n], n being
// here the n_cap the grids and the workspace were sized for.
struct JobIn {
  const afd_job* desc;
  const uint16_t* x;
  const int32_t* ids;
  const float* w;
  uint16_t* out;
  int64_t n;
};

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

// Counter words of one call, in the workspace's num_tiles slot (padded to 256 bytes; num_tiles
// is word 0): the routing launch zeroes words [kCounterWord0, kCounterWord0 + kCounterWords)
// before any later launch of the call uses them.
constexpr int kCounterWord0 = 8, kCounterWords = 32;
constexpr int kGateUpWalkWord = 8;  // the gate_up GEMM's tile counters, one per XCD
constexpr int kDownWalkWord = 16;   // the down GEMM's
constexpr int kArriveWord = 32;     // the reply's arrive counter
inline uint32_t* call_counters(uint8_t* ws, const afd_ws_layout& L) {
  return reinterpret_cast<uint32_t*>(ws + L.num_tiles);
}

// The reply an expert call can carry (afd_moe_ffn_answer): once every output row of the call
// is visible device-wide, *done := value, stored by the last workgroup of the finalize launch
// to finish. arrive counts the finished workgroups. done == nullptr: no reply.
struct Reply {
  uint64_t* done;
  uint64_t value;
  uint32_t* arrive;
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

// Grouped FP8 128x128-block GEMMs (afd_gemm_fp8.hip).
int launch_fp8_gate_up(const afd_moe_cfg& cfg, const afd_expert_weights& wt, uint8_t* ws,
                       const afd_ws_layout& L, const uint8_t* xq, const void* xs,
                       const afd_job* rows_desc, hipStream_t stream);
int launch_fp8_down(const afd_moe_cfg& cfg, const afd_expert_weights& wt, uint8_t* ws,
                    const afd_ws_layout& L, int32_t n, hipStream_t stream);

// Number of compute units of the current device (cached per device).
int device_cu_count();

}  // namespace afd
