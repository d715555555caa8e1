// Quantizers of the expert path on gfx950: MXFP8 / FP8-1x128 activations and the load-time
// MXFP4 / FP8-128x128 weight packers. All are HBM-bound streaming kernels: one lane owns one
// 32-element MX block (16 B fp4 or 32 B fp8 out, 1 scale byte), so every load is a 16-byte
// vector and no cross-lane reduction is needed for MX; FP8 groups of 128 reduce over 4 lanes.
#include "afd_common.h"
#include "afd_internal.h"
#include "afd_quant_dev.h"

namespace afd {


// Logical source row of physical row r when gate and up rows are interleaved in groups of g
// (rows = 2I = [gate; up]): physical 2g*j + q is gate row g*j + q for q < g, else up row.
__device__ __forceinline__ int64_t gate_up_source_row(int64_t r, int64_t rows, int g) {
  int64_t j = r / (2 * g), q = r % (2 * g);
  return q < g ? j * g + q : rows / 2 + j * g + (q - g);
}

// ---------------------------------------------------------------- activation quantizers
// The loops live in afd_quant_dev.h (the router's prep kernel runs them too); these kernels
// give them the whole grid.
template <bool kStageOrder>
__global__ __launch_bounds__(kQuantThreads) void quant_mxfp8_kernel(
    const uint16_t* __restrict__ x, int64_t blocks, int cols, uint8_t* __restrict__ q,
    uint8_t* __restrict__ s) {
  quant_mxfp8_items<kStageOrder>([=](int64_t r) { return x + r * cols; }, blocks, cols, q, s,
                                 blockIdx.x * int64_t(kQuantThreads) + threadIdx.x,
                                 int64_t(gridDim.x) * kQuantThreads);
}

__global__ __launch_bounds__(kQuantThreads) void quant_fp8_1x128_kernel(
    const uint16_t* __restrict__ x, int64_t quarters, int cols, uint8_t* __restrict__ q,
    float* __restrict__ s) {
  quant_fp8_1x128_items([=](int64_t r) { return x + r * cols; }, quarters, cols, q, s,
                        blockIdx.x * int64_t(kQuantThreads) + threadIdx.x,
                        int64_t(gridDim.x) * kQuantThreads);
}

// ---------------------------------------------------------------- MXFP4 weight packer
// One lane per 32-element block of a physical row: 16 bytes of e2m1 codes (one logical
// 16-byte chunk of a B image, since 32 fp4 values = 16 bytes) plus one UE8M0 scale, written
// into the tile image of (matrix, 256-row tile, 128-wide K stage).
__global__ __launch_bounds__(kQuantThreads) void pack_mxfp4_kernel(
    const float* __restrict__ w, int64_t blocks, int rows, int cols, int gate_up,
    uint8_t* __restrict__ out) {
  const int bpr = cols / kMxBlock;
  const int kstages = cols / kImgK, ntiles = rows / kImgBRows;
  for (int64_t b = blockIdx.x * int64_t(kQuantThreads) + threadIdx.x; b < blocks;
       b += int64_t(gridDim.x) * kQuantThreads) {
    int64_t prow = b / bpr;  // physical row over all matrices
    int cb = static_cast<int>(b % bpr);
    int64_t mat = prow / rows;
    int r = static_cast<int>(prow % rows);
    int64_t lr = gate_up ? gate_up_source_row(r, rows, 32) : r;
    const v4f* src = reinterpret_cast<const v4f*>(w + (mat * rows + lr) * cols + cb * kMxBlock);
    float v[32];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      v4f t = src[i];
      v[i * 4] = t[0];
      v[i * 4 + 1] = t[1];
      v[i * 4 + 2] = t[2];
      v[i * 4 + 3] = t[3];
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
    uint32_t code = mx_scale_code(amax, 2);
    float inv = mx_inv_scale(code);
    v4i packed;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t word = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) word |= f32_to_e2m1(v[i * 8 + j] * inv) << (4 * j);
      packed[i] = static_cast<int>(word);
    }
    const int nt = r / kImgBRows, n = r % kImgBRows;
    const int ks = cb / 4, j = cb % 4;
    uint8_t* img = out + ((mat * ntiles + nt) * kstages + ks) * int64_t(kImgB);
    *reinterpret_cast<v4i*>(img + img_b_off(n, j)) = packed;
    img[kImgData + n * 4 + scale_byte(j)] = static_cast<uint8_t>(code);
  }
}

// Physical row of logical row lr when gate and up rows are interleaved in groups of g
// (the inverse of gate_up_source_row).
__device__ __forceinline__ int64_t gate_up_dest_row(int64_t lr, int64_t rows, int g) {
  int64_t half = rows / 2;
  return lr < half ? (lr / g) * 2 * g + lr % g : ((lr - half) / g) * 2 * g + g + (lr - half) % g;
}

// ---------------------------------------------------------------- FP8 128x128 weight packer
// One workgroup per logical 128x128 block: amax over the block, then each lane quantizes 64
// values, one row of an FP8 image (fp8_image_offset). Scales stay in logical block order;
// with gate_up the codes land on the physical rows of the 32-row gate/up interleave.
__global__ __launch_bounds__(kQuantThreads) void pack_fp8_block_kernel(
    const float* __restrict__ w, int rows, int cols, int gate_up, uint8_t* __restrict__ q,
    float* __restrict__ s) {
  __shared__ float red[kQuantThreads / 64];
  const int rbs = rows / kFp8Block, cbs = cols / kFp8Block;
  const int64_t blk = blockIdx.x;
  const int64_t mat = blk / (int64_t(rbs) * cbs);
  const int rb = static_cast<int>((blk / cbs) % rbs), cb = static_cast<int>(blk % cbs);
  const int t = threadIdx.x;
  // lane t: row t/2 of the block, 64 columns starting at (t%2)*64
  const int br = t / 2, bc = (t % 2) * 64;
  const int64_t lrow = int64_t(rb) * kFp8Block + br;
  const int64_t prow = gate_up ? gate_up_dest_row(lrow, rows, 32) : lrow;
  const float* src = w + (mat * rows + lrow) * cols + int64_t(cb) * kFp8Block + bc;
  float v[64];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    v4f x4 = reinterpret_cast<const v4f*>(src)[i];
    v[i * 4] = x4[0];
    v[i * 4 + 1] = x4[1];
    v[i * 4 + 2] = x4[2];
    v[i * 4 + 3] = x4[3];
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 64; ++i) amax = fmaxf(amax, fabsf(v[i]));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  if ((t & 63) == 0) red[t / 64] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float sc = fmaxf(amax, kFp8Eps) / kE4m3Max;
  // the lane's 64 columns are one image row: K stage 2 cb + t % 2 of physical row prow
  uint8_t* img = q + fp8_image_offset(mat, prow, int64_t(cb) * kFp8Block + bc, rows, cols);
  const int rr = static_cast<int>(prow % kImgBRows);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v4i out;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t packed = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b)
        packed |= f32_to_e4m3(clamp_e4m3(v[i * 16 + j * 4 + b] / sc)) << (8 * b);
      out[j] = static_cast<int>(packed);
    }
    *reinterpret_cast<v4i*>(img + img_b_off(rr, i)) = out;
  }
  if (t == 0) s[(mat * rbs + rb) * cbs + cb] = sc;
}

// ---------------------------------------------------------------- checkpoint repack
// Checkpoint MXFP4 experts are already e2m1 codes (two per byte, element 2i in the low
// nibble) with one E8M0 scale per 32: a 32-element block is 16 contiguous code bytes, i.e.
// one 16-byte chunk of a B image. One lane per block of a physical row moves the chunk and
// its scale byte to where afd_pack_mxfp4 would have written them; nothing is requantized.
__global__ __launch_bounds__(kQuantThreads) void repack_mxfp4_kernel(
    const uint8_t* __restrict__ codes, const uint8_t* __restrict__ scales, int64_t blocks,
    int rows, int cols, int gate_up, uint8_t* __restrict__ out) {
  const int bpr = cols / kMxBlock;
  const int kstages = cols / kImgK, ntiles = rows / kImgBRows;
  for (int64_t b = blockIdx.x * int64_t(kQuantThreads) + threadIdx.x; b < blocks;
       b += int64_t(gridDim.x) * kQuantThreads) {
    int64_t prow = b / bpr;
    int cb = static_cast<int>(b % bpr);
    int64_t mat = prow / rows;
    int r = static_cast<int>(prow % rows);
    int64_t src = mat * rows + (gate_up ? gate_up_source_row(r, rows, 32) : r);
    v4i chunk = *reinterpret_cast<const v4i*>(codes + src * (cols / 2) + cb * 16);
    uint8_t code = scales[src * bpr + cb];
    const int nt = r / kImgBRows, n = r % kImgBRows;
    const int ks = cb / 4, j = cb % 4;
    uint8_t* img = out + ((mat * ntiles + nt) * kstages + ks) * int64_t(kImgB);
    *reinterpret_cast<v4i*>(img + img_b_off(n, j)) = chunk;
    img[kImgData + n * 4 + scale_byte(j)] = code;
  }
}

// Checkpoint FP8 block experts: e4m3 rows [mats][rows][cols] moved into the FP8 images, one
// 16-byte chunk a lane (chunk c of physical row r: logical row r's chunk, through the gate/up
// interleave with gate_up).
__global__ __launch_bounds__(kQuantThreads) void repack_fp8_rows_kernel(
    const uint8_t* __restrict__ q, int64_t chunks, int rows, int cols, int gate_up,
    uint8_t* __restrict__ out) {
  const int cpr = cols / 16;
  for (int64_t c = blockIdx.x * int64_t(kQuantThreads) + threadIdx.x; c < chunks;
       c += int64_t(gridDim.x) * kQuantThreads) {
    int64_t prow = c / cpr;
    int j = static_cast<int>(c % cpr);
    int64_t mat = prow / rows;
    int r = static_cast<int>(prow % rows);
    int64_t src = mat * rows + (gate_up ? gate_up_source_row(r, rows, 32) : r);
    uint8_t* img = out + fp8_image_offset(mat, r, int64_t(j) * 16, rows, cols);
    *reinterpret_cast<v4i*>(img + img_b_off(r % kImgBRows, j % 4)) =
        *reinterpret_cast<const v4i*>(q + src * cols + j * 16);
  }
}

int launch_quant_act(const afd_moe_cfg& cfg, const uint16_t* x, int32_t n, uint8_t* q, void* s,
                     hipStream_t stream) {
  if (n == 0) return AFD_OK;
  const int64_t items = int64_t(n) * (cfg.hidden / kMxBlock);
  if (cfg.weight_fmt == AFD_W_MXFP4)
    hipLaunchKernelGGL(quant_mxfp8_kernel<true>, dim3(grid_for(items)), dim3(kQuantThreads), 0,
                       stream, x, items, cfg.hidden, q, static_cast<uint8_t*>(s));
  else
    hipLaunchKernelGGL(quant_fp8_1x128_kernel, dim3(grid_for(items)), dim3(kQuantThreads), 0,
                       stream, x, items, cfg.hidden, q, static_cast<float*>(s));
  AFD_CHECK_LAUNCH();
  return AFD_OK;
}

}  // namespace afd

using namespace afd;

extern "C" int afd_quant_mxfp8(const uint16_t* x, int64_t rows, int32_t cols, uint8_t* q,
                               uint8_t* s, afd_stream_t stream) {
  if (!x || !q || !s || rows < 0) return AFD_ERR_ARG;
  if (cols <= 0 || cols % kMxBlock) return AFD_ERR_SHAPE;
  if (rows == 0) return AFD_OK;
  int64_t blocks = rows * (cols / kMxBlock);
  hipLaunchKernelGGL(quant_mxfp8_kernel<false>, dim3(grid_for(blocks)), dim3(kQuantThreads), 0,
                     static_cast<hipStream_t>(stream), x, blocks, cols, q, s);
  AFD_CHECK_LAUNCH();
  return AFD_OK;
}

extern "C" int afd_quant_fp8_1x128(const uint16_t* x, int64_t rows, int32_t cols, uint8_t* q,
                                   float* s, afd_stream_t stream) {
  if (!x || !q || !s || rows < 0) return AFD_ERR_ARG;
  if (cols <= 0 || cols % kFp8Block) return AFD_ERR_SHAPE;
  if (rows == 0) return AFD_OK;
  int64_t quarters = rows * (cols / kMxBlock);
  hipLaunchKernelGGL(quant_fp8_1x128_kernel, dim3(grid_for(quarters)), dim3(kQuantThreads), 0,
                     static_cast<hipStream_t>(stream), x, quarters, cols, q, s);
  AFD_CHECK_LAUNCH();
  return AFD_OK;
}

extern "C" int afd_pack_mxfp4(const float* w, int64_t mats, int32_t rows, int32_t cols,
                              int32_t gate_up, uint8_t* out, afd_stream_t stream) {
  if (!w || !out || mats < 0) return AFD_ERR_ARG;
  if (rows <= 0 || cols <= 0 || rows % kImgBRows || cols % kImgK) return AFD_ERR_SHAPE;
  if (mats == 0) return AFD_OK;
  int64_t blocks = mats * rows * (cols / kMxBlock);
  hipLaunchKernelGGL(pack_mxfp4_kernel, dim3(grid_for(blocks)), dim3(kQuantThreads), 0,
                     static_cast<hipStream_t>(stream), w, blocks, rows, cols, gate_up ? 1 : 0,
                     out);
  AFD_CHECK_LAUNCH();
  return AFD_OK;
}

extern "C" int afd_pack_fp8_block(const float* w, int64_t mats, int32_t rows, int32_t cols,
                                  int32_t gate_up, uint8_t* q, float* s, afd_stream_t stream) {
  if (!w || !q || !s || mats < 0) return AFD_ERR_ARG;
  if (rows <= 0 || cols <= 0 || rows % kImgBRows || cols % kFp8Block) return AFD_ERR_SHAPE;
  if (mats == 0) return AFD_OK;
  int64_t blocks = mats * (rows / kFp8Block) * (cols / kFp8Block);
  if (blocks > 0x7fffffff) return AFD_ERR_SHAPE;
  hipLaunchKernelGGL(pack_fp8_block_kernel, dim3(static_cast<unsigned>(blocks)),
                     dim3(kQuantThreads), 0, static_cast<hipStream_t>(stream), w, rows, cols,
                     gate_up ? 1 : 0, q, s);
  AFD_CHECK_LAUNCH();
  return AFD_OK;
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

extern "C" int afd_repack_mxfp4(const uint8_t* codes, const uint8_t* scales, int64_t mats,
                                int32_t rows, int32_t cols, int32_t gate_up, uint8_t* out,
                                afd_stream_t stream) {
  if (!codes || !scales || !out || mats < 0) return AFD_ERR_ARG;
  if (!aligned16(codes) || !aligned16(out)) return AFD_ERR_ARG;
  if (rows <= 0 || cols <= 0 || rows % kImgBRows || cols % kImgK) return AFD_ERR_SHAPE;
  if (mats == 0) return AFD_OK;
  int64_t blocks = mats * rows * (cols / kMxBlock);
  hipLaunchKernelGGL(repack_mxfp4_kernel, dim3(grid_for(blocks)), dim3(kQuantThreads), 0,
                     static_cast<hipStream_t>(stream), codes, scales, blocks, rows, cols,
                     gate_up ? 1 : 0, out);
  AFD_CHECK_LAUNCH();
  return AFD_OK;
}

extern "C" int afd_repack_fp8_block(const uint8_t* q, int64_t mats, int32_t rows, int32_t cols,
                                    int32_t gate_up, uint8_t* out, afd_stream_t stream) {
  if (!q || !out || mats < 0) return AFD_ERR_ARG;
  if (!aligned16(q) || !aligned16(out)) return AFD_ERR_ARG;
  if (rows <= 0 || cols <= 0 || rows % kImgBRows || cols % kFp8Block) return AFD_ERR_SHAPE;
  if (mats == 0) return AFD_OK;
  int64_t chunks = mats * rows * (cols / 16);
  hipLaunchKernelGGL(repack_fp8_rows_kernel, dim3(grid_for(chunks)), dim3(kQuantThreads), 0,
                     static_cast<hipStream_t>(stream), q, chunks, rows, cols, gate_up ? 1 : 0,
                     out);
  AFD_CHECK_LAUNCH();
  return AFD_OK;
}
