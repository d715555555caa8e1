// Device loops of the activation quantizers, shared by their kernels (afd_quant.hip) and the
// router's prep kernel (afd_route.hip), which runs one of them beside the expert histogram.
// Every loop is grid-stride over items from `first` with step `stride` (threads). `xrow(r)`
// gives the start of input row r (the rows of a batched call belong to different jobs); the
// outputs q / s are one array over all rows.
#pragma once

#include "afd_common.h"

namespace afd {

constexpr int kQuantThreads = 256;

// workgroups for a grid-stride loop over `items` (at most 32 per CU)
inline int grid_for(int64_t items) {
  int64_t g = (items + kQuantThreads - 1) / kQuantThreads;
  if (g > 8192) g = 8192;
  return static_cast<int>(g < 1 ? 1 : g);
}

// MXFP8: one lane per 32-element block. kStageOrder stores a row's scales as the MX GEMM reads
// them: within each group of 4 blocks (one 128-wide K stage), block j at byte scale_byte(j).
template <bool kStageOrder, typename XRow>
__device__ __forceinline__ void quant_mxfp8_items(XRow xrow, int64_t blocks,
                                                  int cols, uint8_t* __restrict__ q,
                                                  uint8_t* __restrict__ s, int64_t first,
                                                  int64_t stride) {
  const int bpr = cols / kMxBlock;
  for (int64_t b = first; b < blocks; b += stride) {
    int64_t row = b / bpr, cb = b % bpr;
    const v4i* src = reinterpret_cast<const v4i*>(xrow(row) + cb * kMxBlock);
    v4i raw[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) raw[i] = src[i];
    float v[32];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t w = static_cast<uint32_t>(raw[i][j]);
        v[i * 8 + j * 2] = __uint_as_float(w << 16);
        v[i * 8 + j * 2 + 1] = __uint_as_float(w & 0xffff0000u);
      }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
    uint32_t code = mx_scale_code(amax, 8);
    float inv = mx_inv_scale(code);
    v4i out[2];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      out[i / 4][i % 4] = static_cast<int>(
          pk4_e4m3(v[i * 4] * inv, v[i * 4 + 1] * inv, v[i * 4 + 2] * inv, v[i * 4 + 3] * inv));
    v4i* dst = reinterpret_cast<v4i*>(q + row * cols + cb * kMxBlock);
    dst[0] = out[0];
    dst[1] = out[1];
    const int64_t at = kStageOrder ? (cb & ~int64_t(3)) + scale_byte(static_cast<int>(cb & 3)) : cb;
    s[row * bpr + at] = static_cast<uint8_t>(code);
  }
}

// FP8 1x128: 4 consecutive lanes own one group of 128 (32 elements each); amax via two xor
// shuffles, so all lanes of a wavefront iterate together (stride a multiple of 64).
template <typename XRow>
__device__ __forceinline__ void quant_fp8_1x128_items(XRow xrow, int64_t quarters, int cols,
                                                      uint8_t* __restrict__ q,
                                                      float* __restrict__ s, int64_t first,
                                                      int64_t stride) {
  const int qpr = cols / kMxBlock;  // quarter-groups per row
  const int64_t total = (quarters + stride - 1) / stride * stride;
  for (int64_t b = first; b < total; b += stride) {
    bool live = b < quarters;
    int64_t bb = live ? b : 0;
    int64_t row = bb / qpr, cq = bb % qpr;
    const v4i* src = reinterpret_cast<const v4i*>(xrow(row) + cq * kMxBlock);
    float v[32];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v4i r = src[i];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t w = static_cast<uint32_t>(r[j]);
        v[i * 8 + j * 2] = __uint_as_float(w << 16);
        v[i * 8 + j * 2 + 1] = __uint_as_float(w & 0xffff0000u);
      }
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    float sc = fmaxf(amax, kFp8Eps) / kE4m3Max;
    if (!live) continue;
    const float rsc = 1.0f / sc;  // the quotients below are the IEEE v / sc (div_by)
    // hardware conversion (v_cvt_pk_fp8_f32): bit-identical to f32_to_e4m3 on the clamped range
    v4i out[2];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      out[i / 4][i % 4] = static_cast<int>(pk4_e4m3(div_by(v[i * 4], sc, rsc), div_by(v[i * 4 + 1], sc, rsc),
                                                     div_by(v[i * 4 + 2], sc, rsc), div_by(v[i * 4 + 3], sc, rsc)));
    v4i* dst = reinterpret_cast<v4i*>(q + row * cols + cq * kMxBlock);
    dst[0] = out[0];
    dst[1] = out[1];
    if ((cq & 3) == 0) s[row * (cols / kFp8Block) + cq / 4] = sc;
  }
}

}  // namespace afd
