// Grouped GEMMs of the expert FFN with bf16 activations on gfx950 (the activations stay bf16,
// nothing is quantized on the activation side), for both weight formats:
//   W4A16: MXFP4 weights (the tile images afd_pack_mxfp4 writes: 256 rows x 128 K of e2m1
//          codes + UE8M0 scales per image),
//   W8A16: FP8 128x128-block weights (the FP8 images afd_pack_fp8_block writes: 256 rows x
//          64 K of e4m3 per image, + fp32 block scales).
//
//   gate_up: h[p, :] = bf16(act(x_t . Wg_e^T, x_t . Wu_e^T)) for every padded row p of expert
//            e (t = token of the pair at row p), written as the down GEMM's bf16 A images.
//   down:    y[p, :] = bf16(h_p . W2_e^T).
//
// The matrix op is v_mfma_f32_32x32x16_bf16; its weight operand is expanded in registers,
// right before the MFMAs that use it, by v_cvt_scalef32_pk_bf16_fp4 (two e2m1 codes and the
// MX block scale -> two bf16) or v_cvt_scalef32_pk_bf16_fp8 (two e4m3 codes -> two bf16), both
// exact (every value of either format times a power of two is a bf16), so the LDS and HBM keep
// the weights' own 4.25 or 8 bits. The FP8 blocks' fp32 scales are not powers of two: the
// accumulators of a wavefront, whose 128 weight rows lie in one scale block (or, for gate_up,
// one gate and one up block), hold the running sum divided by the current K block's scale,
// and are multiplied by s_prev / s_cur when the K block changes and by the last scale at the
// end; the multiplies run in the wavefront's LDS-read phase, beside the other wavefront's
// MFMAs.
//
// Tiling: a workgroup of 2 x WN wavefronts owns a 128 x (128 WN) output tile; wavefront
// (wm, wn) owns 64 x 128 = 2 x 4 MFMA tiles of 32x32. K stages move HBM -> LDS with direct
// global_load_lds copies in 1 KiB pieces:
//   W4A16: 128 K per stage: the bf16 A block (128 rows x 256 B = 32 KiB, "A16 image") and the
//          tile's WN/2 B images (17 KiB each), in a ring of 2 stages (WN = 4, 132 KiB) or 3;
//   W8A16: 64 K per stage: the bf16 A block (128 rows x 128 B = 16 KiB, "A8 image") and the
//          tile's WN/2 FP8 images (16 KiB each, laid out as an e2m1 B image's data), in a ring
//          of 3 stages (WN = 4: 144 KiB).
// The two wavefronts of a SIMD ping-pong in phases of 64 K (32 MFMAs of 32 clk per wavefront,
// the W4A8 kernel's phase length), so one of them always feeds the matrix pipe while the
// other reads its fragments.
//
// K order inside a 64-wide phase: lane half lk of an MFMA operand holds, in k-step s (0..3),
// K [32 lk + 8 s, +8) of the phase. For the activations that is one 16-byte bf16 chunk of the
// row; for MXFP4 weights dword s of the lane's 16-byte e2m1 chunk (one MX block, one scale),
// for FP8 weights bytes 8 s .. 8 s + 7 of its 32 e4m3 bytes. Both operands use the same K for
// the same (lane half, element), so every product pairs matching elements.
//
// Persistent workgroups, the XCD-aware tile walk (static or dynamic) and the metadata
// prefetch are those of the W4A8 kernels (afd_gemm_mx.hip).
#include <type_traits>

#include "afd_common.h"
#include "afd_internal.h"

namespace afd {

namespace {

enum { kGateUp = 0, kDown = 1, kGateUpParam = 2 };
enum { kWMx = 0, kWFp8 = 1 };  // weight format of the kernel

constexpr int kA16WalkRows = 4;

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

struct A16GemmArgs {
  const uint8_t* a_img;         // down: bf16 A images [row tiles][K / stage K]
  const uint16_t* a_rows;       // gate_up: bf16 token rows [n][K], gathered by sorted_pairs
  const afd_job* rows_desc;     // gate_up: if set, a_rows is its x (read when the kernel runs)
  int topk;                     // gate_up: pairs per token (token of pair p = p / topk)
  uint32_t topk_magic;          // div_magic(topk)
  const uint8_t* b_img;         // MXFP4: B images [E][N/256][K/128]; FP8: images [E][N/256][K/64]
  const float* b_scale;         // FP8: block scales [E][N/128][K/128] (gate blocks, then up)
  const int32_t* sorted_pairs;  // [np] flat pair index per padded row, -1 = pad
  const int32_t* tile_expert;   // [row tiles]
  const int32_t* num_tiles;     // [1]
  const int32_t* padded_offsets;  // [E + 1]
  const int32_t* counts;          // [E]
  uint32_t* walk_ctr;             // zeroed tile counters, XCD x's at x * kWalkCounterStride; nullptr: static walk
  int K, N;
  uint8_t* h_img;  // gate_up out: the down GEMM's bf16 A images [row tiles][N/2 / stage K]
  ActParams act;   // gate_up: the activation
  uint16_t* y;     // down out: bf16 [np][N]
};

// byte offset of logical 16-byte chunk c (0..15, 8 bf16 each) of row r in an A16 image: the
// 16 rows one 16-lane pass of an operand read covers (same logical chunk) land on 16 distinct
// 16-byte bank groups
__host__ __device__ __forceinline__ int img_a16_off(int r, int c) {
  return r * 256 + ((c ^ (r & 15)) << 4);
}

// Stage geometry of a weight format: K per stage, LDS bytes of the A block and of 256 weight
// rows, byte offset of logical chunk c of row r in the A block.
template <int WF>
struct A16Fmt;
template <>
struct A16Fmt<kWMx> {
  static constexpr int kStageK = 128;
  static constexpr int kLdsA = kImgA16;  // 128 rows x 256 B
  static constexpr int kLdsB = kImgB;    // an e2m1 B image with its scales
  static constexpr int kBData = 16;      // data pieces per 256 weight rows
  __host__ __device__ static int a_off(int r, int c) { return img_a16_off(r, c); }
};
template <>
struct A16Fmt<kWFp8> {
  static constexpr int kStageK = 64;
  static constexpr int kLdsA = kImgData;  // 128 rows x 128 B (the W4A8 A image's swizzle)
  static constexpr int kLdsB = kImgF8B;  // an FP8 image: 256 rows x 64 B (the e2m1 B image's swizzle)
  static constexpr int kBData = 16;
  __host__ __device__ static int a_off(int r, int c) { return img_a_off(r, c); }
};

template <int WF, int WN>
struct A16Tile {
  static_assert(WN == 2 || WN == 4, "tiles are 256 or 512 columns wide");
  using F = A16Fmt<WF>;
  static constexpr int kWaves = 2 * WN;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kBM = kBlockM;  // 128 rows = one A block
  static constexpr int kBN = 128 * WN;
  static constexpr int kBImgs = WN / 2;  // 256-row weight blocks per tile
  static constexpr int kStageK = F::kStageK;
  static constexpr int kPhases = kStageK / 64;  // ping-pong phases per stage
  static constexpr int kLdsA = F::kLdsA;
  static constexpr int kStage = kLdsA + kBImgs * F::kLdsB;
  static constexpr int kStages = WF == kWMx && WN == 4 ? 2 : 3;
  static constexpr int kLds = kStages * kStage;
  // per wavefront and stage: kAQ pieces of the A block, kQP data pieces of each 256-row weight
  // block, and (MXFP4, wavefronts below kBImgs) the scale piece of image w
  static constexpr int kAQ = (kLdsA / 1024) / kWaves;
  static constexpr int kARowsPerPiece = 1024 / (kStageK * 2);
  static constexpr int kQP = F::kBData / kWaves;
  static constexpr int kPiecesMin = kAQ + kBImgs * kQP;  // pieces of a wavefront without scales
  static constexpr int kYChunks = kBN / 8;
  static_assert(kBM * kBN * 2 <= kLds, "down epilogue tile must fit the stages");
  static_assert(kLds <= 160 * 1024, "LDS of one CU");
  static_assert(kStages * (kPiecesMin + 1) < 64, "vmcnt is a 6-bit counter");
};

// the 8 e2m1 codes of dword d (element 2i in the low nibble of byte i) times 2^(code - 127),
// as the 8 bf16 of an MFMA operand (element i in half i % 2 of dword i / 2). The instruction
// takes the scale's exponent field as the UE8M0 code, so `scale` is the code shifted into it.
__device__ __forceinline__ v8bf expand_fp4(uint32_t d, float scale) {
  v4i r;
  r[0] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 0));
  r[1] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 1));
  r[2] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 2));
  r[3] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 3));
  return __builtin_bit_cast(v8bf, r);
}

// the 8 e4m3 codes of dwords d0, d1 (element i in byte i % 4 of dword i / 4) as the 8 bf16 of
// an MFMA operand, exactly (scale 2^0)
__device__ __forceinline__ v8bf expand_fp8(uint32_t d0, uint32_t d1) {
  v4i r;
  r[0] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d0, 1.0f, false));
  r[1] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d0, 1.0f, true));
  r[2] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d1, 1.0f, false));
  r[3] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d1, 1.0f, true));
  return __builtin_bit_cast(v8bf, r);
}

// A uniform read of data the kernel never writes (the FP8 block scales), through the scalar
// cache: read through a generic pointer the compiler has to assume a store of the kernel may
// alias it and issues a vector load, whose wait then drains the copies in flight.
__device__ __forceinline__ float load_uniform(const float* p) {
  return *(const __attribute__((address_space(4))) float*)p;
}

template <int WF, int MODE, int WN>
__global__ __launch_bounds__((A16Tile<WF, WN>::kThreads)) void a16_gemm_kernel(A16GemmArgs p) {
  using T = A16Tile<WF, WN>;
  using F = typename T::F;
  constexpr bool kFp8 = WF == kWFp8;
  constexpr int kBM = T::kBM, kBN = T::kBN, kStages = T::kStages, kStage = T::kStage;
  constexpr int kStageK = T::kStageK, kPhases = T::kPhases;
  __shared__ __attribute__((aligned(16))) uint8_t lds[T::kLds];
  const int t = threadIdx.x, lane = t & 63;
  const int w_u = __builtin_amdgcn_readfirstlane(t >> 6);  // wavefront index, scalar
  const int wm = w_u / WN, wn = w_u % WN, lr = lane & 31, lk = lane >> 5;
  const TileWalk<kA16WalkRows> walk(p.num_tiles[0], p.N / kBN, blockIdx.x, gridDim.x, p.walk_ctr);
  __shared__ int claimed[2];
  const int KT = p.K / kStageK;
  const uint32_t lds_base = __builtin_amdgcn_readfirstlane(lds_offset(lds));
  const uint32_t voff = static_cast<uint32_t>(lane) * 16;
  const uint16_t* a_rows = p.a_rows;
  if (MODE != kDown && p.rows_desc != nullptr) a_rows = p.rows_desc->x;
  const int bimg = wn / 2, brow = (wn % 2) * 128;
  // the lane's fragment bases in a stage (see read_phase): A row wm * 64 + lr at chunk 4 lk,
  // weight row brow + lr at chunk lk (MXFP4) or 2 lk (FP8), and (MXFP4) its scale bytes
  const int a_lane = F::a_off(wm * 64 + lr, 4 * lk);
  const int b_lane = T::kLdsA + bimg * F::kLdsB + img_b_off(brow + lr, kFp8 ? 2 * lk : lk);
  const int sb_lane = T::kLdsA + bimg * F::kLdsB + kImgData + 4 * (brow + lr) + 2 * lk;

  // Tile metadata one tile ahead (as the W4A8 kernel). gate_up gathers its A block from the
  // token rows: lane l copies, for its piece q, physical chunk l % C of row R (w kAQ + q) +
  // l / C of the block (C = 16-byte chunks per row, R = rows per piece), i.e. logical chunk
  // (l % C) ^ swizzle(row), from the row's token. Padding rows (-1) read token 0; their
  // results are never stored.
  constexpr int kAChunks = kStageK / 8, kARows = T::kARowsPerPiece;
  int sp_next[T::kAQ], e_next = 0, own_next = -1;
  auto load_next = [&](int ii) {
    int m, nn;
    walk.at_dense(ii, m, nn);
    e_next = p.tile_expert[m];
    own_next = p.sorted_pairs[m * kBM + 64 * wm + lane];
    if constexpr (MODE != kDown) {
#pragma unroll
      for (int q = 0; q < T::kAQ; ++q)
        sp_next[q] = p.sorted_pairs[m * kBM + kARows * (w_u * T::kAQ + q) + lane / kAChunks];
    }
  };
  int e_cur = 0, live_cur = 0;
  uint32_t a_voff[T::kAQ] = {};
  auto decode_next = [&]() {
    e_cur = __builtin_amdgcn_readfirstlane(e_next);
    live_cur = __popcll(__ballot(own_next >= 0));
    if constexpr (MODE != kDown) {
#pragma unroll
      for (int q = 0; q < T::kAQ; ++q) {
        const int r = kARows * (w_u * T::kAQ + q) + lane / kAChunks;
        const int pc = lane % kAChunks;
        const int c = (F::a_off(r, pc) - r * kStageK * 2) >> 4;  // the swizzle is an involution
        const uint32_t tok = sp_next[q] >= 0 ? div_by_magic(static_cast<uint32_t>(sp_next[q]), p.topk_magic) : 0u;
        a_voff[q] = tok * static_cast<uint32_t>(p.K) * 2u + c * 16;
      }
    }
  };
  constexpr bool kEarlyStart = MODE != kDown;
  const uint8_t* a_tile = nullptr;
  const uint8_t* b_tile = nullptr;
  auto copy_tile = [&](int mt, int nt, int64_t e) {
    a_tile = MODE == kDown ? p.a_img + int64_t(mt) * KT * T::kLdsA
                           : reinterpret_cast<const uint8_t*>(a_rows);
    constexpr int64_t kImgBytes = kFp8 ? kImgF8B : kImgB;
    b_tile = p.b_img + (e * (p.N / kImgBRows) + int64_t(nt) * T::kBImgs) * KT * kImgBytes;
  };
  // this wavefront's copies of stage kt into ring slot kt % kStages: its A pieces, its data
  // pieces of every 256-row weight block, and (MXFP4) for w < kBImgs the scale piece of image w
  auto issue = [&](int kt) {
    const uint32_t st = lds_base + static_cast<uint32_t>((kt % kStages) * kStage);
    static_for<T::kAQ>([&](auto qc) {
      constexpr int q = decltype(qc)::value;
      const int off = (w_u * T::kAQ + q) * 1024;
      if constexpr (MODE != kDown)
        lds_dma16(st + off, a_tile + int64_t(kt) * (kStageK * 2), a_voff[q]);
      else
        lds_dma16(st + off, a_tile + int64_t(kt) * T::kLdsA + off, voff);
    });
    static_for<T::kBImgs * T::kQP>([&](auto qc) {
      constexpr int q = decltype(qc)::value;
      constexpr int img = q / T::kQP;
      const int off = (w_u * T::kQP + q % T::kQP) * 1024;
      lds_dma16(st + T::kLdsA + img * F::kLdsB + off, b_tile + (int64_t(img) * KT + kt) * F::kLdsB + off, voff);
    });
    if constexpr (!kFp8) {
      if (w_u < T::kBImgs)
        lds_dma16(st + T::kLdsA + w_u * kImgB + kImgData,
                  b_tile + (int64_t(w_u) * KT + kt) * kImgB + kImgData, voff);
    }
  };
  const int last = KT - 1;

  const bool dynamic = p.walk_ctr != nullptr;
  int i = walk.first, i_next = walk.first + walk.stride;
  if (dynamic) {
    if (t == 0) {
      const uint32_t a = walk.claim_ticket(), b = walk.claim_ticket();
      claimed[0] = walk.resolve(a);
      claimed[1] = walk.resolve(b);
    }
    __syncthreads();
    i = __builtin_amdgcn_readfirstlane(claimed[0]);
    i_next = __builtin_amdgcn_readfirstlane(claimed[1]);
  }
  i = min(i, walk.tiles);
  i_next = min(i_next, walk.tiles);
  uint32_t ticket = 0;
  // A tile's K loop starts with every ring slot filled: stages 0 .. kStages - 1 (clamped to
  // the last stage) are issued before it, either during the previous tile's epilogue (gate_up)
  // or at the start of the tile (down, whose epilogue stages its output through the ring).
  auto issue_first = [&]() {
    static_for<kStages>([&](auto sc) { issue(min(static_cast<int>(decltype(sc)::value), last)); });
  };
  if (i < walk.tiles) {
    load_next(i);
    decode_next();
    if constexpr (kEarlyStart) {
      int mt, nt;
      walk.at_dense(i, mt, nt);
      copy_tile(mt, nt, e_cur);
      issue_first();
    }
  }
  for (int i_after = walk.tiles; i < walk.tiles; i = i_next, i_next = i_after) {
    int mt, nt;
    walk.at_dense(i, mt, nt);
    const bool has_next = i_next < walk.tiles;
    const bool claims = dynamic && t == 0 && has_next;
    const int m0 = mt * kBM, n0 = nt * kBN;
    const int64_t e = e_cur;
    int row_end = 0;
    if constexpr (MODE == kDown) row_end = p.padded_offsets[e] + p.counts[e];
    // this group has a real row (padding rows come last in a segment)
    const bool live_i0 = live_cur > 0;
    if (has_next) load_next(i_next);
    if constexpr (!kEarlyStart) copy_tile(mt, nt, e);

    // FP8 block scales of this wavefront's weight rows (uniform): for gate_up a gate block
    // (j even) and an up block (j odd), for down one block; s_blk[x] points at the block's row
    // of K-block scales
    const int kb_n = p.K / 128;
    const float* s_blk[2] = {nullptr, nullptr};
    float s_run[2] = {1.0f, 1.0f};  // the scales of the K block being accumulated
    float s_next[2] = {1.0f, 1.0f};  // those of the next K block, read one stage ahead
    if constexpr (kFp8) {
      const int row0 = n0 + 128 * wn;  // first weight row of this wavefront
      const float* se = p.b_scale + e * (p.N / 128) * kb_n;
      if constexpr (MODE != kDown) {
        s_blk[0] = se + (row0 / 256) * kb_n;                   // gate rows row0 / 2 + [0, 64)
        s_blk[1] = se + (p.N / 256 + row0 / 256) * kb_n;       // up rows, block I / 128 + ...
      } else {
        s_blk[0] = s_blk[1] = se + (row0 / 128) * kb_n;
      }
      s_run[0] = load_uniform(s_blk[0]);
      s_run[1] = load_uniform(s_blk[1]);
    }

    v16f acc[2][4];
#pragma unroll
    for (int i2 = 0; i2 < 2; ++i2)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int q = 0; q < 16; ++q) acc[i2][j][q] = 0.0f;

    // Fragments of one phase (K 64): A [s][i2] (8 bf16 each); the weights' [j][0] (MXFP4: the
    // lane's e2m1 chunk, with its scale code sb[j]) or [j][0..1] (FP8: its 32 e4m3 bytes)
    struct Frag {
      v4i a[4][2];
      v4i b[4][kFp8 ? 2 : 1];
      uint32_t sb[4];
    };
    Frag f;
    // Every fragment address is one of the lane's bases below, XORed with a few chunk bits and
    // offset by whole rows: A chunk 8 c + 4 lk + s of row r0 (+ 32 i2) sits at
    // (a_lane ^ (8 c + s) << 4 ^ i2 kI2Xor) + i2 kI2Off (the row swizzles leave those chunk
    // bits as they are; row r0 + 32's MXFP4 swizzle equals row r0's, its FP8 one flips chunk
    // bit 2); weight row brow + 32 j + lr's chunk 2 c + lk (MXFP4) or 2 lk + h (FP8) at
    // (b_lane ^ (c or h) << 5 or 4) + 2048 j. A slot's offset leaves the low 8 bits alone, so
    // the XOR is formed after it is added: the addresses are then computed per read instead
    // of being kept as 8-12 loop-invariant registers.
    auto read_phase = [&](int slot, int c) {
      constexpr int kI2Xor = kFp8 ? 64 : 0, kI2Off = kFp8 ? 4096 : 8192;
      const int a0 = slot * kStage + a_lane, b0 = slot * kStage + b_lane;
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i2 = 0; i2 < 2; ++i2)
          f.a[s][i2] = *reinterpret_cast<const v4i*>(lds + ((a0 ^ (((8 * c + s) << 4) | (i2 * kI2Xor))) + i2 * kI2Off));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (kFp8) {
          f.b[j][0] = *reinterpret_cast<const v4i*>(lds + b0 + 2048 * j);
          f.b[j][1] = *reinterpret_cast<const v4i*>(lds + (b0 ^ 16) + 2048 * j);
        } else {
          f.b[j][0] = *reinterpret_cast<const v4i*>(lds + (b0 ^ (c << 5)) + 2048 * j);
          // block 2 c + lk of row n sits at byte scale_byte(2 c + lk) = 2 lk + c
          f.sb[j] = lds[slot * kStage + sb_lane + 128 * j + c];
        }
      }
    };
    // the weight fragment of step (j, s) as 8 bf16
    auto expand = [&](int j, int s, const float (&scale)[4]) -> v8bf {
      if constexpr (kFp8)
        return expand_fp8(static_cast<uint32_t>(f.b[j][s >> 1][2 * (s & 1)]),
                          static_cast<uint32_t>(f.b[j][s >> 1][2 * (s & 1) + 1]));
      else
        return expand_fp4(static_cast<uint32_t>(f.b[j][0][s]), scale[j]);
    };
    // The 32 MFMAs of a phase: 16 steps (j, s), step st expanding the weight fragment of step
    // st + 1 into the other of two register sets while its own 2 MFMAs run, so the converts
    // issue in the MFMAs' shadow. A group whose 64 rows are all padding skips the phase (one
    // uniform branch per phase: branches between the steps, or a second copy of the phase for
    // groups with one live 32-row block, cost more registers than there are).
    auto mma_phase = [&]() {
      float scale[4] = {};
      if constexpr (!kFp8) {
#pragma unroll
        for (int j = 0; j < 4; ++j) scale[j] = __uint_as_float(f.sb[j] << 23);
      }
      v8bf wb[2];
      wb[0] = expand(0, 0, scale);
      static_for<16>([&](auto stc) {
        constexpr int st = decltype(stc)::value, j = st / 4, s = st % 4;
        if constexpr (st + 1 < 16) wb[(st + 1) & 1] = expand((st + 1) / 4, (st + 1) % 4, scale);
        acc[0][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wb[st & 1], __builtin_bit_cast(v8bf, f.a[s][0]),
                                                             acc[0][j], 0, 0, 0);
        acc[1][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wb[st & 1], __builtin_bit_cast(v8bf, f.a[s][1]),
                                                             acc[1][j], 0, 0, 0);
      });
      // issue order: the scale shifts and step 0's expansion, then per step its MFMAs followed
      // by the next step's 4 converts (left to itself the scheduler hoists every expansion
      // ahead of the MFMAs, which needs 64 more registers than there are)
      __builtin_amdgcn_sched_group_barrier(0x2, kFp8 ? 4 : 8, 0);
      static_for<16>([&](auto stc) {
        constexpr int st = decltype(stc)::value;
        __builtin_amdgcn_sched_group_barrier(0x8, 2, 0);
        if constexpr (st + 1 < 16) __builtin_amdgcn_sched_group_barrier(0x2, 4, 0);
      });
    };
    auto mma_live = [&]() {
      if (live_i0) mma_phase();
    };
    // FP8: the second stage of K block kb reads the scales of block kb + 1 (the read phase's
    // own wait covers them); the first stage of block kb > 0 moves the accumulators from the
    // scales of block kb - 1 to those of kb (in the read phase, before its wait)
    auto rescale = [&](int kt) {
      if constexpr (kFp8) {
        if ((kt & 1) && kt + 1 < KT) {
          s_next[0] = load_uniform(s_blk[0] + ((kt + 1) >> 1));
          s_next[1] = load_uniform(s_blk[1] + ((kt + 1) >> 1));
        }
        if (kt > 0 && (kt & 1) == 0) {
          const float s0 = s_next[0], s1 = s_next[1];
          const float r0 = s_run[0] * __builtin_amdgcn_rcpf(s0), r1 = s_run[1] * __builtin_amdgcn_rcpf(s1);
          s_run[0] = s0;
          s_run[1] = s1;
#pragma unroll
          for (int i2 = 0; i2 < 2; ++i2)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
              for (int q = 0; q < 16; ++q) acc[i2][j][q] *= (j & 1) ? r1 : r0;
        }
      }
    };

    // Ping-pong over phases ph = kPhases kt + c (as the W4A8 kernel over stages): group 0
    // reads phase ph + 1 while group 1 multiplies phase ph, and the other way round; every
    // wavefront meets the others at a barrier every phase. At the first phase of stage kt >= 1
    // each group copies its pieces of stage kt + kStages - 1 into the slot of stage kt - 1,
    // which both groups finished reading before the barrier that started the phase (clamped
    // to the last stage: a clamped copy rewrites a slot with its own bytes, and keeps every
    // wavefront's count of copies in flight the same at each wait). Before the barrier after
    // which group 0 reads the first phase of stage kt + 1, both groups have waited for their
    // pieces of it: group 0 after its MFMAs of the phase before, group 1 after its reads of
    // it. The counted waits allow the kStages - 2 later stages in flight (a wavefront that
    // also copies a scale piece waits for one piece more than it needs).
    if constexpr (!kEarlyStart) issue_first();
    wait_vmcnt<(kStages - 1) * T::kPiecesMin>();  // own pieces of stage 0 landed
    __syncthreads();
    const int phases = kPhases * KT;
    if (wm == 0) {
      for (int ph = 0; ph < phases; ++ph) {
        const int kt = ph / kPhases, c = ph % kPhases;
        if (claims && ph == phases - 1) ticket = walk.claim_ticket();
        if (c == 0 && kt >= 1) issue(min(kt + kStages - 1, last));
        read_phase(kt % kStages, c);
        if (c == 0) rescale(kt);
        wait_lds();  // own reads done (copies may be in flight)
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(1);
        mma_live();
        __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_sched_barrier(0);
        if (c == kPhases - 1) wait_vmcnt<(kStages - 2) * T::kPiecesMin>();  // own pieces of stage kt + 1
        __syncthreads();
      }
      __syncthreads();
    } else {
      __syncthreads();
      for (int ph = 0; ph < phases; ++ph) {
        const int kt = ph / kPhases, c = ph % kPhases;
        if (c == 0 && kt >= 1) issue(min(kt + kStages - 1, last));
        read_phase(kt % kStages, c);
        if (c == 0) rescale(kt);
        if (c == kPhases - 1)
          wait_vmcnt_lds<(kStages - 2) * T::kPiecesMin>();  // own reads, own pieces of stage kt + 1
        else
          wait_lds();
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(1);
        mma_live();
        __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
      }
    }
    wait_vmcnt<0>();  // every copy of this tile landed
    if (claims) claimed[0] = walk.resolve(ticket);
    __syncthreads();  // and every wavefront is done reading the stages
    if (has_next) {
      i_after = dynamic ? __builtin_amdgcn_readfirstlane(claimed[0])
                        : min(i_next + walk.stride, walk.tiles);
      decode_next();
      if constexpr (kEarlyStart) {
        int mt2, nt2;
        walk.at_dense(i_next, mt2, nt2);
        copy_tile(mt2, nt2, e_cur);
        issue_first();
      }
    }

    // Accumulator q of tile (i2, j): activation row 64 wm + 32 i2 + lane % 32, output column
    // 128 wn + 32 j + 8 (q / 4) + 4 (lane / 32) + q % 4. Lane half lk holds columns
    // 8 q4 + 4 lk .. + 3 of each 32-column tile; one v_permlane32_swap per pair of bf16 pairs
    // gives lane half lk the whole 16-byte chunks 2 pr + lk (pr = 0, 1), in column order.
    auto chunks_of = [&](const float (&h)[16], v4i (&chunk)[2]) {
      uint32_t hb[4][2];
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        hb[q4][0] = pk_bf16(h[4 * q4], h[4 * q4 + 1]);
        hb[q4][1] = pk_bf16(h[4 * q4 + 2], h[4 * q4 + 3]);
      }
#pragma unroll
      for (int pr = 0; pr < 2; ++pr) {
        const auto d0 = __builtin_amdgcn_permlane32_swap(hb[2 * pr][0], hb[2 * pr + 1][0], false, false);
        const auto d1 = __builtin_amdgcn_permlane32_swap(hb[2 * pr][1], hb[2 * pr + 1][1], false, false);
        chunk[pr] = v4i{static_cast<int>(d0[0]), static_cast<int>(d1[0]), static_cast<int>(d0[1]),
                        static_cast<int>(d1[1])};
      }
    };
    if constexpr (MODE != kDown) {
      // Column tiles j = 2 jj and 2 jj + 1 are the gate and up halves of one 64-row group of
      // interleaved W13: the same 32 intermediate columns n0 / 2 + 64 wn + 32 jj + [0, 32).
      // Their bf16 h chunks go to the down GEMM's A image of row tile mt and K stage
      // column / kStageK, row 64 wm + 32 i2 + lr. FP8: the accumulators take the last K
      // block's scales first.
      const int kt_down = (p.N / 2) / kStageK;  // K stages of the down GEMM
      auto store_h = [&](auto fn) {
        static_for<2>([&](auto ic) {
          constexpr int i2 = decltype(ic)::value;
          const int row = wm * 64 + i2 * 32 + lr;
          static_for<2>([&](auto jjc) {
            constexpr int jj = decltype(jjc)::value;
            float h[16];
#pragma unroll
            for (int q = 0; q < 16; ++q)
              h[q] = fn(acc[i2][2 * jj][q] * s_run[0], acc[i2][2 * jj + 1][q] * s_run[1]);
            v4i chunk[2];
            chunks_of(h, chunk);
            const int col0 = n0 / 2 + 64 * wn + 32 * jj;  // multiple of 32
            uint8_t* img = p.h_img + (int64_t(mt) * kt_down + col0 / kStageK) * T::kLdsA;
#pragma unroll
            for (int pr = 0; pr < 2; ++pr) {
              const int c = (col0 % kStageK) / 8 + 2 * pr + lk;
              *reinterpret_cast<v4i*>(img + F::a_off(row, c)) = chunk[pr];
            }
          });
        });
      };
      if constexpr (MODE == kGateUpParam) {
        if (p.act.act == AFD_ACT_SITU)
          store_h([&](float g, float u) {
            return act_situ(g, u, p.act.a, p.act.inv_a, p.act.l, p.act.inv_l);
          });
        else
          store_h([&](float g, float u) { return act_swiglu_limit(g, u, p.act.l); });
      } else {
        store_h([](float g, float u) { return act_swiglu(g, u); });
      }
    } else {
      // bf16 y rows through LDS so the stores write whole rows (as the W4A8 down GEMM):
      // chunk c of row r at physical chunk c ^ (r % 16); rows [0, nvalid) are real; the
      // stores are non-temporal (y is read once, by the finalize).
      const int nvalid = min(kBM, row_end - m0);
      auto y_chunk = [](int r, int c) { return (r * T::kYChunks + (c ^ (r & 15))) * 16; };
      static_for<2>([&](auto ic) {
        constexpr int i2 = decltype(ic)::value;
        const int row = wm * 64 + i2 * 32 + lr;
        static_for<4>([&](auto jc) {
          constexpr int j = decltype(jc)::value;
          float h[16];
#pragma unroll
          for (int q = 0; q < 16; ++q) h[q] = acc[i2][j][q] * s_run[0];
          v4i chunk[2];
          chunks_of(h, chunk);
#pragma unroll
          for (int pr = 0; pr < 2; ++pr)
            *reinterpret_cast<v4i*>(lds + y_chunk(row, (wn * 128 + j * 32) / 8 + 2 * pr + lk)) = chunk[pr];
        });
      });
      __syncthreads();
#pragma unroll 4
      for (int q = 0; q < kBM * T::kYChunks / T::kThreads; ++q) {
        const int idx = q * T::kThreads + t;
        const int row = idx / T::kYChunks, c = idx % T::kYChunks;
        if (row < nvalid)
          __builtin_nontemporal_store(*reinterpret_cast<const v4i*>(lds + y_chunk(row, c)),
                                      reinterpret_cast<v4i*>(p.y + int64_t(m0 + row) * p.N + n0 + c * 8));
      }
      __syncthreads();
    }
  }
}

template <int WF, int MODE, int WN>
int launch_a16(const A16GemmArgs& p, int max_row_tiles, hipStream_t stream) {
  using T = A16Tile<WF, WN>;
  static const int per_cu = [] {
    int b = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, a16_gemm_kernel<WF, MODE, WN>, T::kThreads,
                                                     0) != hipSuccess ||
        b < 1)
      b = 1;
    return b;
  }();
  const int max_tiles = max_row_tiles * (p.N / T::kBN);
  int grid = device_cu_count() * per_cu;
  if (max_tiles < grid) grid = max_tiles < 1 ? 1 : max_tiles;
  hipLaunchKernelGGL((a16_gemm_kernel<WF, MODE, WN>), dim3(grid), dim3(T::kThreads), 0, stream, p);
  AFD_CHECK_LAUNCH();
  return AFD_OK;
}

template <int WF, int MODE>
int launch_a16_any(const A16GemmArgs& p, int max_row_tiles, hipStream_t stream) {
  if (p.N % A16Tile<WF, 4>::kBN == 0) return launch_a16<WF, MODE, 4>(p, max_row_tiles, stream);
  return launch_a16<WF, MODE, 2>(p, max_row_tiles, stream);
}

A16GemmArgs a16_args(const afd_moe_cfg& cfg, uint8_t* ws, const afd_ws_layout& L) {
  A16GemmArgs p = {};
  p.topk = cfg.topk;
  p.topk_magic = div_magic(cfg.topk);
  p.act = act_params(cfg);
  p.sorted_pairs = reinterpret_cast<const int32_t*>(ws + L.sorted_pairs);
  p.tile_expert = reinterpret_cast<const int32_t*>(ws + L.tile_expert);
  p.num_tiles = reinterpret_cast<const int32_t*>(ws + L.num_tiles);
  p.padded_offsets = reinterpret_cast<const int32_t*>(ws + L.padded_offsets);
  p.counts = reinterpret_cast<const int32_t*>(ws + L.counts);
  return p;
}

template <int WF>
int gate_up(const A16GemmArgs& p, const afd_moe_cfg& cfg, int max_tiles, hipStream_t stream) {
  return cfg.activation != AFD_ACT_SWIGLU ? launch_a16_any<WF, kGateUpParam>(p, max_tiles, stream)
                                         : launch_a16_any<WF, kGateUp>(p, max_tiles, stream);
}

}  // namespace

int launch_a16_gate_up(const afd_moe_cfg& cfg, const afd_expert_weights& wt, uint8_t* ws,
                       const afd_ws_layout& L, const uint16_t* x, const afd_job* rows_desc,
                       hipStream_t stream) {
  A16GemmArgs p = a16_args(cfg, ws, L);
  p.a_rows = x;
  p.rows_desc = rows_desc;
  p.b_img = static_cast<const uint8_t*>(wt.w13);
  p.b_scale = static_cast<const float*>(wt.s13);
  p.walk_ctr = cfg.tile_walk == AFD_WALK_DYNAMIC ? call_counters(ws, L) + kGateUpWalkWord : nullptr;
  p.K = cfg.hidden;
  p.N = 2 * cfg.inter;
  p.h_img = ws + L.hq;
  return cfg.weight_fmt == AFD_W_FP8_BLOCK ? gate_up<kWFp8>(p, cfg, L.max_tiles, stream)
                                           : gate_up<kWMx>(p, cfg, L.max_tiles, stream);
}

int launch_a16_down(const afd_moe_cfg& cfg, const afd_expert_weights& wt, uint8_t* ws,
                    const afd_ws_layout& L, hipStream_t stream) {
  A16GemmArgs p = a16_args(cfg, ws, L);
  p.a_img = ws + L.hq;
  p.b_img = static_cast<const uint8_t*>(wt.w2);
  p.b_scale = static_cast<const float*>(wt.s2);
  p.walk_ctr = cfg.tile_walk == AFD_WALK_DYNAMIC ? call_counters(ws, L) + kDownWalkWord : nullptr;
  p.K = cfg.inter;
  p.N = cfg.hidden;
  p.y = reinterpret_cast<uint16_t*>(ws + L.y);
  return cfg.weight_fmt == AFD_W_FP8_BLOCK ? launch_a16_any<kWFp8, kDown>(p, L.max_tiles, stream)
                                           : launch_a16_any<kWMx, kDown>(p, L.max_tiles, stream);
}

}  // namespace afd
