// Grouped MXFP4-weight x MXFP8-activation GEMMs of the expert FFN on gfx950 scaled MFMA
// (v_mfma_scale_f32_32x32x64_f8f6f4: A e4m3, B e2m1, one UE8M0 scale per lane = per 32 K).
//
//   gate_up: h[p, :] = silu(x_t . Wg_e^T) * (x_t . Wu_e^T) for every padded row p of expert e
//            (t = token of the pair at row p), quantized to MXFP8 in the epilogue.
//   down:    y[p, :] = bf16(h_p . W2_e^T).
//
// Tiling: a workgroup of 4 wavefronts owns a 128 x 256 output tile; wavefront (wm, wn) owns
// 64 x 128 = 2 x 4 MFMA tiles of 32x32 (128 fp32 accumulators per lane). K advances 128 per
// stage (two MFMA k-steps): A 128 rows x 128 B, B 256 rows x 64 B, plus one scale dword
// (4 UE8M0 bytes) per row of each, 33.5 KiB per stage.
//
// Operands move HBM -> LDS with gfx950's direct global_load_lds (no register staging) into a
// ring of 4 stages, three stages ahead of the MFMAs, so a stage has three stages of MFMA time
// to arrive; one barrier per stage. Every wavefront issues the same 10 copies per stage, which
// keeps the vmcnt arithmetic of the waits uniform. LDS rows are XOR-swizzled by 16-byte chunk
// (the copies place each lane's chunk at its swizzled slot) so the ds_read_b128 of 8
// consecutive rows hit 8 distinct bank groups.
//
// The workgroups are persistent: grid = resident workgroups, tile index strides by the grid,
// and the number of row tiles is read from device memory (the router wrote it), so no host
// round trip is needed. Tile index order is (row tile, column tile) with column tiles fastest,
// so consecutive workgroups (which the dispatcher spreads over the 8 XCDs) split a weight
// tile's columns across XCDs and each expert's weights are fetched from HBM once.
#include "afd_common.h"
#include "afd_internal.h"

namespace afd {

constexpr int kBM = kBlockM;  // 128
constexpr int kBN = 256;
constexpr int kBK = 128;
constexpr int kThreads = 256;
constexpr int kAStage = kBM * kBK;       // fp8 A bytes per stage
constexpr int kBStage = kBN * kBK / 2;   // fp4 B bytes per stage
constexpr int kSAStage = kBM * 4;
constexpr int kSBStage = kBN * 4;
constexpr int kStage = kAStage + kBStage + kSAStage + kSBStage;
constexpr int kStages = 4;
constexpr int kCopiesPerStage = 10;  // per wavefront: 4 A + 4 B + 1 A-scale + 1 B-scale
constexpr int kLdsBytes = kStages * kStage;
constexpr int kHStride = 132;  // fp32 stride of the gate_up epilogue tile (128 + 4)
constexpr int kYStride = 264;  // bf16 stride of the down epilogue tile (256 + 8)
static_assert(kBM * kHStride * 4 <= kLdsBytes, "gate_up epilogue tile must fit the stages");
static_assert(kBM * kYStride * 2 <= kLdsBytes, "down epilogue tile must fit the stages");

enum { kGateUp = 0, kDown = 1 };

struct MxGemmArgs {
  const uint8_t* a;             // gate_up: xq [n][K]; down: hq [np][K]
  const uint8_t* as;            // UE8M0 [rows][K/32]
  const int32_t* sorted_pairs;  // [np] flat pair index per padded row, -1 = pad
  const int32_t* tile_expert;   // [row tiles]
  const int32_t* num_tiles;     // [1]
  const uint8_t* b;             // e2m1 [E][N][K/2]
  const uint8_t* bs;            // UE8M0 [E][N][K/32]
  int K, N, topk;
  uint8_t* hq;   // gate_up out: e4m3 [np][N/2]
  uint8_t* hs;   // gate_up out: UE8M0 [np][N/64]
  uint16_t* y;   // down out: bf16 [np][N]
};

__device__ __forceinline__ int a_off(int r, int c) { return r * 128 + ((c ^ (r & 7)) << 4); }
__device__ __forceinline__ int b_off(int n, int c) { return n * 64 + ((c ^ ((n >> 1) & 3)) << 4); }

template <int MODE>
__device__ __forceinline__ int64_t a_row(const MxGemmArgs& p, int m) {
  if (MODE == kGateUp) {
    int sp = p.sorted_pairs[m];
    return sp >= 0 ? sp / p.topk : 0;
  }
  return m;
}

template <int MODE>
__global__ __launch_bounds__(kThreads) void mx_gemm_kernel(MxGemmArgs p) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kLdsBytes];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1, lr = lane & 31, lk = lane >> 5;
  const int ntn = p.N / kBN;
  const int tiles = p.num_tiles[0] * ntn;
  const int KT = p.K / kBK;
  const int64_t a_ld = p.K, s_ld = p.K / 32, b_ld = p.K / 2;

  for (int tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
    const int mt = tile / ntn, nt = tile % ntn;
    const int m0 = mt * kBM, n0 = nt * kBN;
    const int64_t e = p.tile_expert[mt];

    // Per-lane 32-bit source offsets of this tile's copies (fixed over K; the K position
    // goes into the uniform base). Copy q of wavefront w fills 1 KiB: A rows w*32+q*8+lane/8,
    // B rows w*64+q*16+lane/4; each lane loads the logical chunk that belongs at its
    // swizzled LDS slot.
    uint32_t voff_a[4], voff_b[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      int r = wave * 32 + q * 8 + (lane >> 3);
      voff_a[q] = static_cast<uint32_t>(a_row<MODE>(p, m0 + r) * a_ld) +
                  (static_cast<uint32_t>((lane & 7) ^ (lane >> 3)) << 4);
      int n = wave * 64 + q * 16 + (lane >> 2);
      voff_b[q] = static_cast<uint32_t>((e * p.N + n0 + n) * b_ld) +
                  (static_cast<uint32_t>((lane & 3) ^ ((lane >> 3) & 3)) << 4);
    }
    const uint32_t voff_sa = static_cast<uint32_t>(a_row<MODE>(p, m0 + wave * 32 + (lane & 31)) * s_ld);
    const uint32_t voff_sb = static_cast<uint32_t>((e * p.N + n0 + wave * 64 + lane) * s_ld);
    const uint32_t lds_base = __builtin_amdgcn_readfirstlane(lds_offset(lds));
    const int w_u = __builtin_amdgcn_readfirstlane(wave);

    auto issue = [&](int kt) {
      const uint32_t st = lds_base + static_cast<uint32_t>((kt % kStages) * kStage);
      const uint8_t* abase = p.a + kt * kBK;
      const uint8_t* bbase = p.b + kt * (kBK / 2);
#pragma unroll
      for (int q = 0; q < 4; ++q) lds_dma16(st + (w_u * 32 + q * 8) * 128, abase, voff_a[q]);
#pragma unroll
      for (int q = 0; q < 4; ++q)
        lds_dma16(st + kAStage + (w_u * 64 + q * 16) * 64, bbase, voff_b[q]);
      if (lane < 32) lds_dma4(st + kAStage + kBStage + w_u * 32 * 4, p.as + kt * 4, voff_sa);
      lds_dma4(st + kAStage + kBStage + kSAStage + w_u * 64 * 4, p.bs + kt * 4, voff_sb);
    };

    v16f acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.0f;

    auto compute = [&](int s) {
      const uint8_t* base = lds + s * kStage;
      const uint32_t* sa = reinterpret_cast<const uint32_t*>(base + kAStage + kBStage);
      const uint32_t* sb = sa + kBM;
      uint32_t sav[2], sbv[4];
#pragma unroll
      for (int i = 0; i < 2; ++i) sav[i] = sa[wm * 64 + i * 32 + lr];
#pragma unroll
      for (int j = 0; j < 4; ++j) sbv[j] = sb[wn * 128 + j * 32 + lr];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        v8i af[2], bf[4];
        // 8-bit operand of the f8f6f4 MFMA: lane half h holds K [16h, 16h+16) in bytes 0-15
        // and K [32+16h, 32+16h+16) in bytes 16-31 of the 64-wide k-step; the fp4 operand
        // holds K [32h, 32h+32) contiguously, and the scale of lane x+32b covers K block b.
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          int r = wm * 64 + i * 32 + lr;
          v4i lo = *reinterpret_cast<const v4i*>(base + a_off(r, ks * 4 + lk));
          v4i hi = *reinterpret_cast<const v4i*>(base + a_off(r, ks * 4 + 2 + lk));
          af[i] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          int n = wn * 128 + j * 32 + lr;
          v4i v = *reinterpret_cast<const v4i*>(base + kAStage + b_off(n, ks * 2 + lk));
          bf[j] = v8i{v[0], v[1], v[2], v[3], 0, 0, 0, 0};
        }
        const int sh = 8 * (ks * 2 + lk);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          int sca = static_cast<int>((sav[i] >> sh) & 0xffu);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            int scb = static_cast<int>((sbv[j] >> sh) & 0xffu);
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                af[i], bf[j], acc[i][j], 0 /*A e4m3*/, 4 /*B e2m1*/, 0, sca, 0, scb);
          }
        }
      }
    };

    wait_vmcnt<0>();  // the previous tile's epilogue stores
#pragma unroll
    for (int s = 0; s < kStages - 1; ++s)
      if (s < KT) issue(s);
    for (int kt = 0; kt < KT; ++kt) {
      // stage kt's copies are done when at most the later stages' copies are outstanding
      if (kt + 2 < KT)
        wait_vmcnt<2 * kCopiesPerStage>();
      else if (kt + 1 < KT)
        wait_vmcnt<kCopiesPerStage>();
      else
        wait_vmcnt<0>();
      // every wavefront's copies of stage kt have landed, and every wavefront is done with
      // stage kt-1, whose buffer the next copy overwrites
      __syncthreads();
      if (kt + kStages - 1 < KT) issue(kt + kStages - 1);
      compute(kt % kStages);
    }
    __syncthreads();  // the epilogue reuses the stage buffers

    if (MODE == kGateUp) {
      // SwiGLU in registers: column subtiles (0,1) and (2,3) are the (gate, up) halves of
      // one 64-row group of interleaved W13, i.e. the same 32 intermediate columns.
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
            hl[row * kHStride + col] = __fdividef(g, 1.0f + __expf(-g)) * u;
          }
      __syncthreads();
      const int inter = p.N / 2;
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        int b = t + half * kThreads;  // 128 rows x 4 MX blocks
        int row = b >> 2, cb = b & 3;
        int grow = m0 + row;
        const float* src = hl + row * kHStride + cb * 32;
        float v[32];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          v4f x4 = reinterpret_cast<const v4f*>(src)[i];
          v[i * 4] = x4[0];
          v[i * 4 + 1] = x4[1];
          v[i * 4 + 2] = x4[2];
          v[i * 4 + 3] = x4[3];
        }
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
        uint32_t code = mx_scale_code(amax, 8);
        float inv = mx_inv_scale(code);
        v4i out[2];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          out[i / 4][i % 4] = static_cast<int>(pk4_e4m3(v[i * 4] * inv, v[i * 4 + 1] * inv,
                                                        v[i * 4 + 2] * inv, v[i * 4 + 3] * inv));
        if (p.sorted_pairs[grow] >= 0) {
          v4i* dst = reinterpret_cast<v4i*>(p.hq + int64_t(grow) * inter + n0 / 2 + cb * 32);
          dst[0] = out[0];
          dst[1] = out[1];
          p.hs[int64_t(grow) * (inter / 32) + n0 / 64 + cb] = static_cast<uint8_t>(code);
        }
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
        int idx = q * kThreads + t;  // 128 rows x 32 chunks of 8 bf16
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

template <int MODE>
static int persistent_grid(int max_tiles) {
  static int per_cu = 0;  // resident workgroups per CU (registers and LDS decide)
  if (per_cu == 0) {
    int b = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, mx_gemm_kernel<MODE>, kThreads, 0) !=
            hipSuccess ||
        b < 1)
      b = 1;
    per_cu = b;
  }
  int g = device_cu_count() * per_cu;
  return max_tiles < g ? (max_tiles < 1 ? 1 : max_tiles) : g;
}

int launch_mx_gate_up(const afd_moe_cfg& cfg, const afd_expert_weights& wt, uint8_t* ws,
                      const afd_ws_layout& L, int32_t n, hipStream_t stream) {
  (void)n;
  MxGemmArgs p;
  p.a = ws + L.xq;
  p.as = ws + L.xs;
  p.sorted_pairs = reinterpret_cast<const int32_t*>(ws + L.sorted_pairs);
  p.tile_expert = reinterpret_cast<const int32_t*>(ws + L.tile_expert);
  p.num_tiles = reinterpret_cast<const int32_t*>(ws + L.num_tiles);
  p.b = static_cast<const uint8_t*>(wt.w13);
  p.bs = static_cast<const uint8_t*>(wt.s13);
  p.K = cfg.hidden;
  p.N = 2 * cfg.inter;
  p.topk = cfg.topk;
  p.hq = ws + L.hq;
  p.hs = ws + L.hs;
  p.y = nullptr;
  int grid = persistent_grid<kGateUp>(L.max_tiles * (p.N / kBN));
  hipLaunchKernelGGL(mx_gemm_kernel<kGateUp>, dim3(grid), dim3(kThreads), 0, stream, p);
  AFD_CHECK_LAUNCH();
  return AFD_OK;
}

int launch_mx_down(const afd_moe_cfg& cfg, const afd_expert_weights& wt, uint8_t* ws,
                   const afd_ws_layout& L, int32_t n, hipStream_t stream) {
  (void)n;
  MxGemmArgs p;
  p.a = ws + L.hq;
  p.as = ws + L.hs;
  p.sorted_pairs = reinterpret_cast<const int32_t*>(ws + L.sorted_pairs);
  p.tile_expert = reinterpret_cast<const int32_t*>(ws + L.tile_expert);
  p.num_tiles = reinterpret_cast<const int32_t*>(ws + L.num_tiles);
  p.b = static_cast<const uint8_t*>(wt.w2);
  p.bs = static_cast<const uint8_t*>(wt.s2);
  p.K = cfg.inter;
  p.N = cfg.hidden;
  p.topk = cfg.topk;
  p.hq = nullptr;
  p.hs = nullptr;
  p.y = reinterpret_cast<uint16_t*>(ws + L.y);
  int grid = persistent_grid<kDown>(L.max_tiles * (p.N / kBN));
  hipLaunchKernelGGL(mx_gemm_kernel<kDown>, dim3(grid), dim3(kThreads), 0, stream, p);
  AFD_CHECK_LAUNCH();
  return AFD_OK;
}

}  // namespace afd
