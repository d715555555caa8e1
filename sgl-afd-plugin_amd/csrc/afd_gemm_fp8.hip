// Grouped FP8-e4m3 GEMMs with 128x128-block fp32 weight scales and 1x128 fp32 activation
// scales (the block-FP8 expert format) on gfx950 MFMA (v_mfma_f32_32x32x64_f8f6f4, e4m3 x
// e4m3, unscaled).
//
// A K stage is exactly one 128-wide scale block: the two MFMA k-steps of a stage accumulate
// into a per-stage partial, which is then folded into the running accumulator with
// acc += partial * (s_a[row] * s_w[block]) - the exact block-scaled product, computed in fp32.
//
// Tiling as in the MXFP4 kernel (128 x 256 per workgroup, 2 x 2 wavefronts of 64 x 128), with
// a 32 KiB fp8 B stage; two stages take ~97 KiB of LDS, one workgroup per CU. W13 rows are
// interleaved gate/up in groups of 32 as in the MXFP4 layout, so SwiGLU happens in registers;
// W13 scales stay in logical block order ([gate blocks; up blocks]), so each wavefront's
// column subtiles j = 0, 2 use the gate block scale and j = 1, 3 the up block scale.
#include "afd_common.h"
#include "afd_internal.h"

namespace afd {
namespace fp8 {

constexpr int kBM = kBlockM;  // 128
constexpr int kBN = 256;
constexpr int kBK = 128;
constexpr int kThreads = 256;
constexpr int kAStage = kBM * kBK;  // 16 KiB
constexpr int kBStage = kBN * kBK;  // 32 KiB
constexpr int kSAStage = kBM * 4;
constexpr int kSBStage = 128;  // 2 floats used, padded
constexpr int kStage = kAStage + kBStage + kSAStage + kSBStage;
constexpr int kLdsBytes = 2 * kStage;
constexpr int kHStride = 132;
constexpr int kYStride = 264;
static_assert(kBM * kHStride * 4 <= kLdsBytes, "epilogue tile must fit");

enum { kGateUp = 0, kDown = 1 };

struct Fp8GemmArgs {
  const uint8_t* a;   // gate_up: xq [n][K]; down: hq [np][K]
  const float* as;    // [rows][K/128]
  const int32_t* sorted_pairs;
  const int32_t* tile_expert;
  const int32_t* num_tiles;
  const uint8_t* b;   // e4m3 [E][N][K] (gate_up rows interleaved by 32)
  const float* bs;    // [E][N/128][K/128] logical block order
  int K, N, topk;
  uint8_t* hq;        // gate_up out e4m3 [np][N/2]
  float* hs;          // gate_up out [np][N/256]
  uint16_t* y;        // down out bf16 [np][N]
};

__device__ __forceinline__ int row_off(int r, int c) { return r * 128 + ((c ^ (r & 7)) << 4); }

template <int MODE>
__device__ __forceinline__ int64_t a_row(const Fp8GemmArgs& p, int m) {
  if (MODE == kGateUp) {
    int sp = p.sorted_pairs[m];
    return sp >= 0 ? sp / p.topk : 0;
  }
  return m;
}

template <int MODE>
__global__ __launch_bounds__(kThreads) void fp8_gemm_kernel(Fp8GemmArgs p) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kLdsBytes];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1, lr = lane & 31, lk = lane >> 5;
  const int ntn = p.N / kBN;
  const int tiles = p.num_tiles[0] * ntn;
  const int KT = p.K / kBK;
  const int64_t a_ld = p.K, sa_ld = p.K / kBK, b_ld = p.K;
  const int kb = p.K / kBK;        // scale blocks along K
  const int nb_all = p.N / kBK;    // scale blocks along N

  for (int tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
    const int mt = tile / ntn, nt = tile % ntn;
    const int m0 = mt * kBM, n0 = nt * kBN;
    const int64_t e = p.tile_expert[mt];

    const uint8_t* a_src[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      int r = j * 32 + (t >> 3);
      a_src[j] = p.a + a_row<MODE>(p, m0 + r) * a_ld + (t & 7) * 16;
    }
    const uint8_t* b_src[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      int n = j * 32 + (t >> 3);
      b_src[j] = p.b + (e * p.N + n0 + n) * b_ld + (t & 7) * 16;
    }
    const float* sa_src = p.as + a_row<MODE>(p, m0 + (t & (kBM - 1))) * sa_ld;
    // the two weight scale blocks this tile touches
    int sblk = 0;
    if (MODE == kGateUp)
      sblk = (t == 0) ? n0 / 256 : (nb_all / 2 + n0 / 256);
    else
      sblk = n0 / 128 + (t & 1);
    const float* sb_src = p.bs + (e * nb_all + sblk) * kb;

    v4i ra[4], rb[8];
    float rsa = 0.0f, rsb = 0.0f;
    auto load = [&](int kt) {
      const int k0 = kt * kBK;
#pragma unroll
      for (int j = 0; j < 4; ++j) ra[j] = *reinterpret_cast<const v4i*>(a_src[j] + k0);
#pragma unroll
      for (int j = 0; j < 8; ++j) rb[j] = *reinterpret_cast<const v4i*>(b_src[j] + k0);
      if (t < kBM) rsa = sa_src[kt];
      if (t < 2) rsb = sb_src[kt];
    };
    auto store = [&](int s) {
      uint8_t* base = lds + s * kStage;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        int r = j * 32 + (t >> 3);
        *reinterpret_cast<v4i*>(base + row_off(r, t & 7)) = ra[j];
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        int n = j * 32 + (t >> 3);
        *reinterpret_cast<v4i*>(base + kAStage + row_off(n, t & 7)) = rb[j];
      }
      float* sa = reinterpret_cast<float*>(base + kAStage + kBStage);
      if (t < kBM) sa[t] = rsa;
      if (t < 2) sa[kBM + t] = rsb;
    };

    v16f acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.0f;
    const v16f zero = {};

    load(0);
    store(0);
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
      if (kt + 1 < KT) load(kt + 1);
      const uint8_t* base = lds + (kt & 1) * kStage;
      const float* sa = reinterpret_cast<const float*>(base + kAStage + kBStage);
      v16f part[2][4];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        v8i af[2], bf[4];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          int r = wm * 64 + i * 32 + lr;
          int c0 = ks * 4 + lk * 2;
          v4i lo = *reinterpret_cast<const v4i*>(base + row_off(r, c0));
          v4i hi = *reinterpret_cast<const v4i*>(base + row_off(r, c0 + 1));
          af[i] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          int n = wn * 128 + j * 32 + lr;
          int c0 = ks * 4 + lk * 2;
          v4i lo = *reinterpret_cast<const v4i*>(base + kAStage + row_off(n, c0));
          v4i hi = *reinterpret_cast<const v4i*>(base + kAStage + row_off(n, c0 + 1));
          bf[j] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            part[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                af[i], bf[j], ks == 0 ? zero : part[i][j], 0, 0, 0, 0, 0, 0);
      }
      // fold the stage's partial with its block scales
      float sbw[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) sbw[j] = MODE == kGateUp ? sa[kBM + (j & 1)] : sa[kBM + wn];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        float sav[16];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          v4f s4 = *reinterpret_cast<const v4f*>(sa + wm * 64 + i * 32 + g * 8 + lk * 4);
          sav[g * 4] = s4[0];
          sav[g * 4 + 1] = s4[1];
          sav[g * 4 + 2] = s4[2];
          sav[g * 4 + 3] = s4[3];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int q = 0; q < 16; ++q)
            acc[i][j][q] = fmaf(part[i][j][q], sav[q] * sbw[j], acc[i][j][q]);
      }
      if (kt + 1 < KT) store((kt + 1) & 1);
      __syncthreads();
    }

    if (MODE == kGateUp) {
      float* hl = reinterpret_cast<float*>(lds);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
#pragma unroll
          for (int q = 0; q < 16; ++q) {
            int row = wm * 64 + i * 32 + (q >> 2) * 8 + lk * 4 + (q & 3);
            int col = wn * 64 + jj * 32 + lr;
            float g = acc[i][2 * jj][q], u = acc[i][2 * jj + 1][q];
            hl[row * kHStride + col] = g / (1.0f + expf(-g)) * u;
          }
      __syncthreads();
      // one 1x128 group per row: 2 lanes per row, 64 values each
      const int inter = p.N / 2;
      const int row = t >> 1, half = t & 1;
      const int grow = m0 + row;
      const float* src = hl + row * kHStride + half * 64;
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
      amax = fmaxf(amax, __shfl_xor(amax, 1));
      const float sc = fmaxf(amax, kFp8Eps) / kE4m3Max;
      if (p.sorted_pairs[grow] >= 0) {
        uint8_t* dst = p.hq + int64_t(grow) * inter + n0 / 2 + half * 64;
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
          reinterpret_cast<v4i*>(dst)[i] = out;
        }
        if (half == 0) p.hs[int64_t(grow) * (inter / kBK) + n0 / 256] = sc;
      }
      __syncthreads();
    } else {
      uint16_t* yl = reinterpret_cast<uint16_t*>(lds);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int q = 0; q < 16; ++q) {
            int row = wm * 64 + i * 32 + (q >> 2) * 8 + lk * 4 + (q & 3);
            int col = wn * 128 + j * 32 + lr;
            yl[row * kYStride + col] = f32_to_bf16(acc[i][j][q]);
          }
      __syncthreads();
#pragma unroll 4
      for (int q = 0; q < 16; ++q) {
        int idx = q * kThreads + t;
        int row = idx >> 5, c = idx & 31;
        int grow = m0 + row;
        if (p.sorted_pairs[grow] >= 0)
          *reinterpret_cast<v4i*>(p.y + int64_t(grow) * p.N + n0 + c * 8) =
              *reinterpret_cast<const v4i*>(yl + row * kYStride + c * 8);
      }
      __syncthreads();
    }
  }
}

static int persistent_grid(int max_tiles) {
  int g = device_cu_count();  // ~97 KiB of LDS: one workgroup per CU
  return max_tiles < g ? (max_tiles < 1 ? 1 : max_tiles) : g;
}

}  // namespace fp8

int launch_fp8_gate_up(const afd_moe_cfg& cfg, const afd_expert_weights& wt, uint8_t* ws,
                       const afd_ws_layout& L, int32_t n, hipStream_t stream) {
  (void)n;
  fp8::Fp8GemmArgs p;
  p.a = ws + L.xq;
  p.as = reinterpret_cast<const float*>(ws + L.xs);
  p.sorted_pairs = reinterpret_cast<const int32_t*>(ws + L.sorted_pairs);
  p.tile_expert = reinterpret_cast<const int32_t*>(ws + L.tile_expert);
  p.num_tiles = reinterpret_cast<const int32_t*>(ws + L.num_tiles);
  p.b = static_cast<const uint8_t*>(wt.w13);
  p.bs = static_cast<const float*>(wt.s13);
  p.K = cfg.hidden;
  p.N = 2 * cfg.inter;
  p.topk = cfg.topk;
  p.hq = ws + L.hq;
  p.hs = reinterpret_cast<float*>(ws + L.hs);
  p.y = nullptr;
  int grid = fp8::persistent_grid(L.max_tiles * (p.N / fp8::kBN));
  hipLaunchKernelGGL(fp8::fp8_gemm_kernel<fp8::kGateUp>, dim3(grid), dim3(fp8::kThreads), 0,
                     stream, p);
  AFD_CHECK_LAUNCH();
  return AFD_OK;
}

int launch_fp8_down(const afd_moe_cfg& cfg, const afd_expert_weights& wt, uint8_t* ws,
                    const afd_ws_layout& L, int32_t n, hipStream_t stream) {
  (void)n;
  fp8::Fp8GemmArgs p;
  p.a = ws + L.hq;
  p.as = reinterpret_cast<const float*>(ws + L.hs);
  p.sorted_pairs = reinterpret_cast<const int32_t*>(ws + L.sorted_pairs);
  p.tile_expert = reinterpret_cast<const int32_t*>(ws + L.tile_expert);
  p.num_tiles = reinterpret_cast<const int32_t*>(ws + L.num_tiles);
  p.b = static_cast<const uint8_t*>(wt.w2);
  p.bs = static_cast<const float*>(wt.s2);
  p.K = cfg.inter;
  p.N = cfg.hidden;
  p.topk = cfg.topk;
  p.hq = nullptr;
  p.hs = nullptr;
  p.y = reinterpret_cast<uint16_t*>(ws + L.y);
  int grid = fp8::persistent_grid(L.max_tiles * (p.N / fp8::kBN));
  hipLaunchKernelGGL(fp8::fp8_gemm_kernel<fp8::kDown>, dim3(grid), dim3(fp8::kThreads), 0,
                     stream, p);
  AFD_CHECK_LAUNCH();
  return AFD_OK;
}

}  // namespace afd
