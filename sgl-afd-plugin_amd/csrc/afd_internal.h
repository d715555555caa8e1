// Declarations shared by the translation units of libafd (not part of the C ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/afd.h"

namespace afd {

constexpr int kMaxLocalExperts = 256;
constexpr int kMaxTopk = 32;
constexpr int kBlockM = 128;  // row tile of the grouped GEMMs; expert segments pad to it


// Routing of the job's pairs into the workspace; with x, the activation quantization into
// ws.xq / ws.xs (MXFP8 in stage order, or FP8 1x128, by cfg.weight_fmt) runs beside the
// expert histogram. `mid` (optional) is recorded between the two launches.
// Activation quantization as the expert call applies it (MXFP8 with stage-order scales, or
// FP8 1x128, by cfg.weight_fmt) into q / s.
int launch_quant_act(const afd_moe_cfg& cfg, const uint16_t* x, int32_t n, uint8_t* q, void* s,
                     hipStream_t stream);

int launch_route_quant(const int32_t* ids, int32_t n, const afd_moe_cfg& cfg, uint8_t* ws,
                       const afd_ws_layout& L, const uint16_t* x, hipStream_t stream,
                       hipEvent_t mid);

// Grouped MXFP4 GEMMs (afd_gemm_mx.hip).
// xq / xs: the quantized activation rows [n][H] and their scales (the workspace's, or the
// caller's for afd_moe_ffn_q)
int launch_mx_gate_up(const afd_moe_cfg& cfg, const afd_expert_weights& wt, uint8_t* ws,
                      const afd_ws_layout& L, const uint8_t* xq, const void* xs, int32_t n,
                      hipStream_t stream);
int launch_mx_down(const afd_moe_cfg& cfg, const afd_expert_weights& wt, uint8_t* ws,
                   const afd_ws_layout& L, int32_t n, hipStream_t stream);

// Grouped FP8 128x128-block GEMMs (afd_gemm_fp8.hip).
int launch_fp8_gate_up(const afd_moe_cfg& cfg, const afd_expert_weights& wt, uint8_t* ws,
                       const afd_ws_layout& L, const uint8_t* xq, const void* xs, int32_t n,
                       hipStream_t stream);
int launch_fp8_down(const afd_moe_cfg& cfg, const afd_expert_weights& wt, uint8_t* ws,
                    const afd_ws_layout& L, int32_t n, hipStream_t stream);

// Number of compute units of the current device (cached per device).
int device_cu_count();

}  // namespace afd
