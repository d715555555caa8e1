// Grouped FP8-e4m3 GEMMs with 128x128-block fp32 weight scales and 1x128 fp32 activation
// scales (W8A8, the block-FP8 expert format) on gfx950 MFMA (v_mfma_scale_f32_32x32x64_f8f6f4
// with unit scales, e4m3 x e4m3).
//
//   gate_up: h[p, :] = act(x_t . Wg_e^T, x_t . Wu_e^T) for every padded row p of expert e
//            (t = token of the pair at row p), quantized to e4m3 with one fp32 scale per 1x128
//            group: the down GEMM's A operand (FP8 images of 128 rows x 64 K) and its scales.
//   down:    y[p, :] = bf16(h_p . W2_e^T).
//
// Block scales: the 64-K stages 2 kb and 2 kb + 1 make up scale block kb of both operands,
// with s_kb = s_x[row, kb] * s_w[block, kb]; the result is sum_kb s_kb * P_kb, P_kb the
// block's unscaled MFMA sum. The accumulators hold R_kb = (sum_{k <= kb} s_k P_k) / s_kb: at
// the first stage of block kb > 0 they are multiplied by s_{kb-1} / s_kb (in the wavefront's
// LDS-read phase, beside the other wavefront's MFMAs), the MFMAs then add P_kb, and the
// epilogue multiplies by the last s. No second set of registers holds partial sums; the
// result rounds differently from folding each block separately by about one fp32 rounding
// per block (relative 2^-24 each). The MFMA operands are swapped (weights first, activations
// second), so a lane's accumulators all belong to one activation row and s_kb is one value
// per 32x32 tile and lane.
//
// Tiling: a workgroup of 8 wavefronts owns a 256 x 256 output tile (the router pads this
// format's expert segments to 256 rows, so a row tile is one expert's); wavefront (wm, wn)
// owns 64 x 128 = 2 x 4 MFMA tiles of 32x32 (128 fp32 accumulators per lane), so per MFMA a
// lane reads 1.5 fragments of 32 bytes from LDS. The square tile needs the fewest operand
// bytes per MAC that 8 x 128 accumulators allow (a stage moves 33 KiB for 4 M MACs, against
// 40.5 KiB for a 128 x 512 tile): the copies into LDS, not the matrix pipe, bound these
// GEMMs. K advances 64 per stage (one MFMA k-step). A stage is the A block (256 rows x 64 B
// of e4m3: gate_up gathers the token rows through sorted_pairs, down copies one FP8 image of
// h), the tile's FP8 weight image (16 KiB, contiguous in HBM: afd_pack_fp8_block's layout)
// and the 256 activation rows' scales of the stage's K block; everything moves HBM -> LDS
// with gfx950's direct global_load_lds (1 KiB pieces, the scales as 4-byte words), into a
// ring of 3 stages (down: 4). Both operands keep the e2m1 B image's swizzled 64-byte rows (img_b_off)
// in LDS: the 16-byte chunks an MFMA operand read takes from 16 consecutive rows fall on 16
// distinct 16-byte bank groups. The two wavefronts of a SIMD ping-pong between reading a
// stage's fragments and running its 8 MFMAs (as the W4A8 and W4A16 kernels), and the
// persistent workgroups walk the tiles XCD by XCD (TileWalk), statically or by claims.
#include <type_traits>

#include "afd_common.h"
#include "afd_internal.h"

namespace afd {
namespace fp8 {

// gate_up with SwiGLU, gate_up with an activation that takes constants (SiTU, or SwiGLU with
// a limit), down
enum { kGateUp = 0, kDown = 1, kGateUpParam = 2 };

// Tile walk blocks of 8 row tiles: a weight slice is shared by 8 row tiles of its expert in L2.
constexpr int kWalkRows = 8;

struct Fp8GemmArgs {
  const uint8_t* a;          // gate_up: token rows xq [n][K]; down: h images [row tiles][K/64]
  const float* as;           // gate_up: xs [n][K/128]; down: hs [row tiles][K/128][128]
  const afd_job* rows_desc;  // gate_up: if set, a / as are its xq / xs (read when the kernel runs)
  int topk;
  uint32_t topk_magic;  // div_magic(topk)
  const uint8_t* b;     // FP8 images [E][N/256][K/64] (gate_up rows interleaved gate/up by 32)
  const float* bs;      // [E][N/128][K/128] in logical block order (gate blocks, then up)
  const int32_t* sorted_pairs;    // [np] flat pair index per padded row, -1 = pad
  const int32_t* tile_expert;     // [row tiles]
  const int32_t* num_tiles;       // [1]
  const int32_t* padded_offsets;  // [E + 1]
  const int32_t* counts;          // [E]
  uint32_t* walk_ctr;             // [8] zeroed tile counters (one per XCD); nullptr: static walk
  int K, N;
  ActParams act;  // gate_up: the activation
  uint8_t* hq;    // gate_up out: h images [row tiles][N/2/64]
  float* hs;      // gate_up out: h scales [row tiles][N/2/128][128]
  uint16_t* y;    // down out: bf16 [np][N]
};

// The tile: 256 activation rows (two 128-row blocks of one expert: the router pads this
// format's expert segments to 256 rows) x 256 weight rows. Eight wavefronts, (wm, wn) =
// (w / 2, w % 2), own 64 x 128 each; wavefronts w and w + 4 share a SIMD, so the ping-pong
// groups are w < 4 (rows 0-127) and w >= 4 (rows 128-255).
struct Tile {
  static constexpr int kWaves = 8;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kBM = kFp8BlockM;
  static constexpr int kBN = 256;
  // LDS stage: A block (256 rows x 64 B), the weight image (256 rows x 64 B), the 256
  // activation rows' fp32 scales of the stage's K block
  static constexpr int kBOff = kImgF8B;
  static constexpr int kAScale = 2 * kImgF8B;
  static constexpr int kStage = kAScale + kBM * 4;
  // ring slots: gate_up 3 (its scale table takes the rest of the LDS), down 4 (its epilogue
  // tile covers the ring; one more stage in flight measured 3% faster)
  template <int MODE>
  static constexpr int stages() { return MODE == 1 ? 4 : 3; }
  static constexpr int kRing = 3 * kStage;
  // down: its epilogue's bf16 tile over the ring. gate_up: after the ring, the epilogue's
  // per-row amax of each column wavefront, [2][256 rows], then the tile's activation-row
  // scales for every K block (the scale table, filled once per tile; see the kernel)
  static constexpr int kYBytes = kBM * kBN * 2;
  static constexpr int kDownLds = 4 * kStage > kYBytes ? 4 * kStage : kYBytes;
  static constexpr int kAmax = kRing;
  static constexpr int kTab = kAmax + 2 * kBM * 4;
  static constexpr int kTabMaxQ = 7;  // table pieces per wavefront: K up to 7168
  static constexpr int kGateUpLds = kTab + kWaves * kTabMaxQ * 1024;  // 256 rows x 14 chunks
  static constexpr int kLds = kDownLds > kGateUpLds ? kDownLds : kGateUpLds;
  // per wavefront and stage: 2 pieces of the A block and 2 of the weight image; wavefronts
  // 0-3 also copy the scale words of rows [64 w, 64 w + 64)
  static constexpr int kAQ = (kImgF8B / 1024) / kWaves;
  static constexpr int kQP = (kImgF8B / 1024) / kWaves;
  static constexpr int kPiecesMin = kAQ + kQP;  // pieces of a wavefront without scales
  static constexpr int kYChunks = kBN / 8;
  static_assert(kBM == 256 && kAQ * kWaves * 1024 == kImgF8B, "pieces cover a stage");
  static_assert((kStage & 255) == 0, "slot offsets leave the fragment addresses' low 8 bits alone");
  static_assert(kLds + 256 <= 160 * 1024, "LDS of one CU");
  template <int MODE>
  static constexpr int lds_bytes() { return MODE == 1 ? kDownLds : kGateUpLds; }
  static_assert(4 * (kPiecesMin + 1) < 64, "vmcnt is a 6-bit counter");
};

// A uniform read of data the kernel never writes (the weight block scales), through the
// scalar cache: a vector load's wait would drain the copies in flight.
__device__ __forceinline__ float load_uniform(const float* p) {
  return *(const __attribute__((address_space(4))) float*)p;
}

template <int MODE>
__global__ __launch_bounds__(Tile::kThreads) void fp8_gemm_kernel(Fp8GemmArgs p) {
  using T = Tile;
  constexpr int kBM = T::kBM, kBN = T::kBN, kStages = T::stages<MODE>(), kStage = T::kStage;
  __shared__ __attribute__((aligned(16))) uint8_t lds[T::lds_bytes<MODE>()];
  const int t = threadIdx.x, lane = t & 63;
  const int w_u = __builtin_amdgcn_readfirstlane(t >> 6);  // wavefront index, scalar
  const int wm = w_u >> 1, wn = w_u & 1, lr = lane & 31, lk = lane >> 5;
  const TileWalk<kWalkRows> walk(p.num_tiles[0], p.N / kBN, blockIdx.x, gridDim.x, p.walk_ctr);
  __shared__ int claimed[2];  // the claimed walk positions lane 0 publishes (as in the MX kernel)
  const int KT = p.K / kF8K;
  const int kb_n = p.K / 128;  // scale blocks along K
  const uint32_t lds_base = __builtin_amdgcn_readfirstlane(lds_offset(lds));
  const uint32_t voff = static_cast<uint32_t>(lane) * 16;
  const uint8_t* a_rows = p.a;
  const float* a_scales = p.as;
  if (MODE != kDown && p.rows_desc != nullptr) {
    a_rows = p.rows_desc->xq;
    a_scales = static_cast<const float*>(p.rows_desc->xs);
  }
  // fragment bases of the lane in a stage: A row 64 wm + lr and weight row 128 wn + lr, each
  // at logical chunk lk (the operand's first 16 bytes; its second 16 are logical chunk lk + 2,
  // i.e. the address with bit 5 flipped). Rows + 32 i keep the swizzle.
  const int a_lane = img_b_off(wm * 64 + lr, lk);
  const int b_lane = T::kBOff + img_b_off(wn * 128 + lr, lk);
  // gate_up's activation-row scales: with K a multiple of 512 up to 7168, every row's K-block
  // scales (K / 128 words, contiguous in xs) are copied once per tile into the scale table;
  // otherwise wavefronts 0-3 copy the 256 rows' words of each stage's K block into its slot.
  // The table holds 16-byte chunk c (the scales of K blocks 4 c .. 4 c + 3) of row r at
  // (256 c + r) * 16, so the 32 rows an operand read takes fill consecutive 16-byte units (no
  // bank conflicts); wavefront w copies chunks c = 2 q + w / 4 of rows 64 (w % 4) + lane.
  const int tab_chunks = kb_n / 4;
  const bool table = MODE != kDown && kb_n % 4 == 0 && (tab_chunks + 1) / 2 <= T::kTabMaxQ;
  const bool copies_scales = w_u < 4 && !table;
  auto tab_off = [&](int r, int c) { return T::kTab + (c * kBM + r) * 16; };

  // Tile metadata one tile ahead (as the W4A8 kernel). gate_up gathers its A block from the
  // token rows: lane l copies, for its piece q (16 rows), physical chunk l % 4 of row
  // 16 (w kAQ + q) + l / 4 of the block, i.e. logical chunk (l % 4) ^ swizzle(row), from the
  // row's token; the scale-copying wavefront w < 4 copies the word of row 64 w + l. Padding
  // rows (-1) read token 0; their results are never stored.
  int sp_next[T::kAQ + 2], e_next = 0, own_next = -1;
  auto load_next = [&](int ii) {
    int m, nn;
    walk.at_dense(ii, m, nn);
    e_next = p.tile_expert[m];
    own_next = p.sorted_pairs[m * kBM + 64 * wm + lane];
    if constexpr (MODE != kDown) {
#pragma unroll
      for (int q = 0; q < T::kAQ; ++q)
        sp_next[q] = p.sorted_pairs[m * kBM + 16 * (w_u * T::kAQ + q) + (lane >> 2)];
      sp_next[T::kAQ] = p.sorted_pairs[m * kBM + 64 * (w_u & 3) + lane];
      sp_next[T::kAQ + 1] = p.sorted_pairs[m * kBM + 64 * (w_u & 3) + lane];
    }
  };
  int e_cur = 0, live_cur = 0;
  uint32_t a_voff[T::kAQ] = {}, s_voff = 0, t_voff = 0;
  auto decode_next = [&]() {
    e_cur = __builtin_amdgcn_readfirstlane(e_next);
    live_cur = __popcll(__ballot(own_next >= 0));  // real rows of this group, a scalar
    if constexpr (MODE != kDown) {
      auto token = [&](int sp) {
        return sp >= 0 ? div_by_magic(static_cast<uint32_t>(sp), p.topk_magic) : 0u;
      };
#pragma unroll
      for (int q = 0; q < T::kAQ; ++q) {
        const int r = 16 * (w_u * T::kAQ + q) + (lane >> 2);
        const int c = (img_b_off(r, lane & 3) - r * kF8K) >> 4;  // the swizzle is an involution
        a_voff[q] = token(sp_next[q]) * static_cast<uint32_t>(p.K) + c * 16;
      }
      s_voff = token(sp_next[T::kAQ]) * static_cast<uint32_t>(kb_n * 4);
      t_voff = token(sp_next[T::kAQ + 1]) * static_cast<uint32_t>(kb_n * 4);
    }
  };
  // gate_up starts the next tile's copies right after its own K loop: its epilogue works from
  // registers and an LDS area past the ring. down's epilogue stages its output through the
  // ring, so it starts them at the tile start.
  constexpr bool kEarlyStart = MODE != kDown;
  const uint8_t* a_tile = nullptr;
  const float* s_tile = nullptr;
  const uint8_t* b_tile = nullptr;
  auto copy_tile = [&](int mt, int nt, int64_t e) {
    a_tile = MODE != kDown ? a_rows : a_rows + int64_t(mt) * KT * kImgF8B;
    s_tile = MODE != kDown ? a_scales : a_scales + int64_t(mt) * kb_n * kBM;
    b_tile = p.b + (e * (p.N / kImgBRows) + nt) * KT * int64_t(kImgF8B);
  };
  // this wavefront's copies of stage kt into ring slot kt % kStages: its A pieces, its
  // weight pieces, and (wavefronts 0-3) scale words
  auto issue = [&](int kt) {
    const uint32_t st = lds_base + static_cast<uint32_t>((kt % kStages) * kStage);
    static_for<T::kAQ>([&](auto qc) {
      constexpr int q = decltype(qc)::value;
      const int off = (w_u * T::kAQ + q) * 1024;
      if constexpr (MODE != kDown)
        lds_dma16(st + off, a_tile + int64_t(kt) * kF8K, a_voff[q]);
      else
        lds_dma16(st + off, a_tile + int64_t(kt) * kImgF8B + off, voff);
    });
    static_for<T::kQP>([&](auto qc) {
      constexpr int q = decltype(qc)::value;
      const int off = (w_u * T::kQP + q) * 1024;
      lds_dma16(st + T::kBOff + off, b_tile + int64_t(kt) * kImgF8B + off, voff);
    });
    if (copies_scales) {
      if constexpr (MODE != kDown)
        lds_dma4(st + T::kAScale + w_u * 256, s_tile + (kt >> 1), s_voff);
      else
        lds_dma4(st + T::kAScale + w_u * 256, s_tile + (kt >> 1) * kBM + 64 * w_u, lane * 4u);
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
  uint32_t ticket = 0;  // lives across the tile loop (no write to its register waits for it)
  // A tile's K loop starts with every ring slot filled: stages 0 .. kStages - 1 (clamped to
  // the last stage) are issued before it, during the previous tile's epilogue (gate_up) or at
  // the start of the tile (down).
  // (gate_up with the scale table: the tile's table pieces first, so the wait for stage 0
  // covers them; the previous tile's K loop, the table's only reader, has ended by then)
  auto issue_first = [&]() {
    if (MODE != kDown && table) {
      for (int c = w_u >> 2; c < tab_chunks; c += 2)
        lds_dma16(lds_base + static_cast<uint32_t>(tab_off(64 * (w_u & 3), c)), s_tile,
                  t_voff + static_cast<uint32_t>(c * 16));
    }
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
    const bool claims = dynamic && t == 0 && has_next;  // publishes the tile after next
    const int m0 = mt * kBM, n0 = nt * kBN;
    const int64_t e = e_cur;
    // down: the expert's pairs fill its first rows; rows below row_end are real
    int row_end = 0;
    if constexpr (MODE == kDown) row_end = p.padded_offsets[e] + p.counts[e];
    // 32-row blocks of this group with a real row (padding rows come last in a segment)
    const bool live_i0 = live_cur > 0, live_i1 = live_cur > 32;
    if (has_next) load_next(i_next);
    if constexpr (!kEarlyStart) copy_tile(mt, nt, e);

    // The weight block scales of this wavefront's 128 weight rows (uniform): gate_up a gate
    // block (tiles j even) and an up block (j odd), down one block for both; s_blk[x] points
    // at the block's row of K-block scales. sw0, sw1: those of the K block being accumulated,
    // swn0, swn1: of the next one, read a block ahead. The activation rows' scales of the
    // K block (sx0, sx1: lane rows 64 wm + lr and + 32), read from the stage's scale words.
    const float* s_blk[2];
    {
      const int row0 = n0 + 128 * wn;
      const float* se = p.bs + e * (p.N / 128) * kb_n;
      if constexpr (MODE != kDown) {
        s_blk[0] = se + (row0 / 256) * kb_n;
        s_blk[1] = se + (p.N / 256 + row0 / 256) * kb_n;
      } else {
        s_blk[0] = s_blk[1] = se + (row0 / 128) * kb_n;
      }
    }
    // (named scalars, not arrays: arrays written in the branches below end up in scratch)
    float sw0 = load_uniform(s_blk[0]), sw1 = load_uniform(s_blk[1]);
    float swn0 = sw0, swn1 = sw1;
    float sx0 = 1.0f, sx1 = 1.0f;

    v16f acc[2][4];
#pragma unroll
    for (int i2 = 0; i2 < 2; ++i2)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int q = 0; q < 16; ++q) acc[i2][j][q] = 0.0f;

    // The fragments of one stage: an 8-bit operand's lane half h holds K [16 h, 16 h + 16) in
    // bytes 0-15 and K [32 + 16 h, + 16) in bytes 16-31, i.e. logical chunks h and h + 2 of
    // the row's 64 bytes.
    v8i fa[2], fb[4];
    auto read_stage = [&](int kt) {
      const int a0 = (kt % kStages) * kStage + a_lane, b0 = (kt % kStages) * kStage + b_lane;
#pragma unroll
      for (int i2 = 0; i2 < 2; ++i2) {
        const v4i lo = *reinterpret_cast<const v4i*>(lds + a0 + 2048 * i2);
        const v4i hi = *reinterpret_cast<const v4i*>(lds + (a0 ^ 32) + 2048 * i2);
        fa[i2] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const v4i lo = *reinterpret_cast<const v4i*>(lds + b0 + 2048 * j);
        const v4i hi = *reinterpret_cast<const v4i*>(lds + (b0 ^ 32) + 2048 * j);
        fb[j] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
    };
    // At the first stage of K block kb (even kt), in the read phase: the block's activation
    // scales from the slot, the factors s_{kb-1} / s_kb of the accumulators, and the next
    // block's weight scales read ahead. The multiplies themselves run in the MFMA phase, each
    // tile's 16 right before its MFMA: the tile's previous MFMA finished a phase ago, and the
    // next tile's multiplies issue beside this tile's MFMA.
    float r00 = 1.0f, r01 = 1.0f, r10 = 1.0f, r11 = 1.0f;
    v4f xc0 = {}, xc1 = {};  // scale-table chunks of the lane's two rows (see block_scales)
    int kb_next = 0;  // the K block whose weight scales swn0, swn1 hold
    auto block_scales = [&](int kt) {
      float x0, x1;
      if (MODE != kDown && table) {
        // one 16-byte read per row brings the scales of 4 K blocks; they shift down a lane of
        // the vector per block
        if (((kt >> 1) & 3) == 0) {
          xc0 = *reinterpret_cast<const v4f*>(lds + tab_off(wm * 64 + lr, kt >> 3));
          xc1 = *reinterpret_cast<const v4f*>(lds + tab_off(wm * 64 + 32 + lr, kt >> 3));
        }
        x0 = xc0[0];
        x1 = xc1[0];
        xc0 = v4f{xc0[1], xc0[2], xc0[3], xc0[3]};
        xc1 = v4f{xc1[1], xc1[2], xc1[3], xc1[3]};
      } else {
        const float* sxs = reinterpret_cast<const float*>(lds + (kt % kStages) * kStage + T::kAScale);
        x0 = sxs[wm * 64 + lr];
        x1 = sxs[wm * 64 + 32 + lr];
      }
      r00 = (sx0 * sw0) * __builtin_amdgcn_rcpf(x0 * swn0);
      r01 = (sx0 * sw1) * __builtin_amdgcn_rcpf(x0 * swn1);
      r10 = (sx1 * sw0) * __builtin_amdgcn_rcpf(x1 * swn0);
      r11 = (sx1 * sw1) * __builtin_amdgcn_rcpf(x1 * swn1);
      sw0 = swn0;
      sw1 = swn1;
      sx0 = x0;
      sx1 = x1;
      kb_next = min(kb_next + 1, kb_n - 1);
      swn0 = load_uniform(s_blk[0] + kb_next);
      swn1 = load_uniform(s_blk[1] + kb_next);
    };
    // the stage's 8 MFMAs (D[weight row][activation row]), 32-row blocks of padding skipped;
    // with `moved`, each tile's accumulators take their factor first
    auto mma_stage = [&](bool moved) {
      static_for<2>([&](auto i2c) {
        constexpr int i2 = decltype(i2c)::value;
        if (i2 == 0 ? live_i0 : live_i1) {
          static_for<4>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            if (moved) {
              const float r = i2 == 0 ? ((j & 1) ? r01 : r00) : ((j & 1) ? r11 : r10);
#pragma unroll
              for (int q = 0; q < 16; ++q) acc[i2][j][q] *= r;
            }
            acc[i2][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                fb[j], fa[i2], acc[i2][j], 0 /*e4m3*/, 0 /*e4m3*/, 0, 127 /*x1*/, 0, 127 /*x1*/);
            // keeps each tile's multiplies after the previous MFMA (hoisted, they would need
            // registers for all 128 products at once)
            if (moved) __builtin_amdgcn_sched_barrier(0);
          });
        }
      });
    };
    // Ping-pong over stages: group 0 reads stage kt + 1 while group 1 multiplies stage kt, and
    // the other way round; every wavefront meets the others at a barrier every half stage. At
    // stage kt >= 1 each group copies its pieces of stage kt + 2 into the slot of stage
    // kt - 1, which both groups finished reading before the barrier that started this read
    // phase (clamped to the last stage: a clamped copy rewrites a slot with its own bytes, and
    // keeps every wavefront's count of copies in flight the same at each wait). Before the
    // barrier after which group 0 reads stage kt + 1, both groups have waited for their pieces
    // of it: group 0 after its MFMAs of stage kt, group 1 after its reads of stage kt. The
    // counted waits allow one later stage in flight (a wavefront that also copies scale words
    // waits for one piece more than it needs).
    if constexpr (!kEarlyStart) issue_first();
    wait_vmcnt<(kStages - 1) * T::kPiecesMin>();  // own pieces of stage 0 landed
    __syncthreads();
    // The loops take two stages per iteration (KT is even), the K block's first with the
    // accumulators' factor and its second without, so neither MFMA phase branches on it (the
    // factor of block 0 multiplies zeros).
    if (w_u < 4) {
      auto phase = [&](int kt, auto first_c) {
        constexpr bool kFirst = decltype(first_c)::value;
        // the claim rides on the last stage, whose end waits for every copy anyway
        if (!kFirst && claims && kt == last) ticket = walk.claim_ticket();
        if (kt >= 1) issue(min(kt + kStages - 1, last));
        read_stage(kt);
        if constexpr (kFirst) block_scales(kt);
        wait_lds();  // own reads done (copies may be in flight)
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(1);
        mma_stage(kFirst);
        __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt<(kStages - 2) * T::kPiecesMin>();  // own pieces of stage kt + 1
        __syncthreads();
      };
      for (int kt = 0; kt < KT; kt += 2) {
        phase(kt, std::true_type{});
        phase(kt + 1, std::false_type{});
      }
      __syncthreads();
    } else {
      __syncthreads();
      auto phase = [&](int kt, auto first_c) {
        constexpr bool kFirst = decltype(first_c)::value;
        if (kt >= 1) issue(min(kt + kStages - 1, last));
        read_stage(kt);
        if constexpr (kFirst) block_scales(kt);
        wait_vmcnt_lds<(kStages - 2) * T::kPiecesMin>();  // own reads, own pieces of stage kt + 1
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(1);
        mma_stage(kFirst);
        __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
      };
      for (int kt = 0; kt < KT; kt += 2) {
        phase(kt, std::true_type{});
        phase(kt + 1, std::false_type{});
      }
    }
    // R_last * s_last
    {
      const float l00 = sx0 * sw0, l01 = sx0 * sw1, l10 = sx1 * sw0, l11 = sx1 * sw1;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          acc[0][j][q] *= (j & 1) ? l01 : l00;
          acc[1][j][q] *= (j & 1) ? l11 : l10;
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
    // 128 wn + 32 j + 8 (q / 4) + 4 (lane / 32) + q % 4.
    if constexpr (MODE != kDown) {
      // Column tiles j = 2 jj and 2 jj + 1 are the gate and up halves of one 64-row group of
      // interleaved W13: h columns n0 / 2 + 64 wn + 32 jj + [0, 32), 16 values of each row in
      // this lane and 16 in lane ^ 32. The tile's 128 h columns are one 1x128 group per row:
      // the row's amax over both column wavefronts goes through an LDS area past the ring. Each
      // lane half then assembles 16 contiguous codes with one exchange and stores them into
      // the down GEMM's A image (row tile mt, K stage column / 64); the group's scale goes
      // to the scale table.
      const int inter = p.N / 2;
      float* amax_l = reinterpret_cast<float*>(lds + T::kAmax);
      auto quant_store = [&](auto fn) {
        float h[2][2][16];
#pragma unroll
        for (int i2 = 0; i2 < 2; ++i2) {
          float m = 0.0f;
#pragma unroll
          for (int jj = 0; jj < 2; ++jj)
#pragma unroll
            for (int q = 0; q < 16; ++q) {
              h[i2][jj][q] = fn(acc[i2][2 * jj][q], acc[i2][2 * jj + 1][q]);
              m = fmaxf(m, fabsf(h[i2][jj][q]));
            }
          m = fmaxf(m, xor32(m, lk));
          if (lk == 0) amax_l[wn * kBM + wm * 64 + i2 * 32 + lr] = m;
        }
        __syncthreads();
#pragma unroll
        for (int i2 = 0; i2 < 2; ++i2) {
          const int row = wm * 64 + i2 * 32 + lr;
          const float amax = fmaxf(amax_l[row], amax_l[kBM + row]);
          const float sc = fmaxf(amax, kFp8Eps) / kE4m3Max;
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) {
            uint32_t d[4];
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4)
              d[q4] = pk4_e4m3(h[i2][jj][4 * q4] / sc, h[i2][jj][4 * q4 + 1] / sc,
                               h[i2][jj][4 * q4 + 2] / sc, h[i2][jj][4 * q4 + 3] / sc);
            // lane half 0 takes columns 0-15 (its d0, d1 and the partner's), half 1 columns
            // 16-31 (the partner's d2, d3 and its own)
            const uint32_t p0 = swap_halves(d[2], d[0], lk);
            const uint32_t p1 = swap_halves(d[3], d[1], lk);
            v4i chunk;
            chunk[0] = static_cast<int>(lk ? p0 : d[0]);
            chunk[1] = static_cast<int>(lk ? d[2] : p0);
            chunk[2] = static_cast<int>(lk ? p1 : d[1]);
            chunk[3] = static_cast<int>(lk ? d[3] : p1);
            const int col0 = n0 / 2 + 64 * wn + 32 * jj;  // multiple of 32
            uint8_t* img = p.hq + (int64_t(mt) * (inter / kF8K) + col0 / kF8K) * kImgF8B;
            *reinterpret_cast<v4i*>(img + img_b_off(row, (col0 % kF8K) / 16 + lk)) = chunk;
            if (jj == 0 && wn == 0 && lk == 0)
              p.hs[(int64_t(mt) * (inter / 128) + col0 / 128) * kBM + row] = sc;
          }
        }
      };
      if constexpr (MODE == kGateUpParam) {
        if (p.act.act == AFD_ACT_SITU)
          quant_store([&](float g, float u) {
            return act_situ(g, u, p.act.a, p.act.inv_a, p.act.l, p.act.inv_l);
          });
        else
          quant_store([&](float g, float u) { return act_swiglu_limit(g, u, p.act.l); });
      } else {
        quant_store([](float g, float u) { return act_swiglu(g, u); });
      }
      // the amax area is read before the next tile's epilogue writes it again: every
      // wavefront passes the next K loop's barriers in between
    } else {
      // bf16 y rows through LDS (chunk c of row r at physical chunk c ^ (r % 16)), so the
      // stores write whole rows. Lane half lk holds columns 8 q4 + 4 lk .. + 3 of each
      // 32-column tile; trading halves with v_permlane32_swap leaves lane half lk with whole
      // 16-byte chunks 2 pr + lk, in column order. Rows [0, nvalid) of this tile are real;
      // the stores are non-temporal (y is read once, by the finalize).
      const int nvalid = min(kBM, row_end - m0);
      auto y_chunk = [](int r, int c) { return (r * T::kYChunks + (c ^ (r & 15))) * 16; };
      static_for<2>([&](auto ic) {
        constexpr int i2 = decltype(ic)::value;
        const int row = wm * 64 + i2 * 32 + lr;
        static_for<4>([&](auto jc) {
          constexpr int j = decltype(jc)::value;
          uint32_t h[4][2];
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) {
            h[q4][0] = pk_bf16(acc[i2][j][4 * q4], acc[i2][j][4 * q4 + 1]);
            h[q4][1] = pk_bf16(acc[i2][j][4 * q4 + 2], acc[i2][j][4 * q4 + 3]);
          }
#pragma unroll
          for (int pr = 0; pr < 2; ++pr) {
            const auto d0 = __builtin_amdgcn_permlane32_swap(h[2 * pr][0], h[2 * pr + 1][0], false, false);
            const auto d1 = __builtin_amdgcn_permlane32_swap(h[2 * pr][1], h[2 * pr + 1][1], false, false);
            const v4i chunk = {static_cast<int>(d0[0]), static_cast<int>(d1[0]), static_cast<int>(d0[1]),
                               static_cast<int>(d1[1])};
            *reinterpret_cast<v4i*>(lds + y_chunk(row, (wn * 128 + j * 32) / 8 + 2 * pr + lk)) = chunk;
          }
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

template <int MODE>
static int launch(const Fp8GemmArgs& p, int max_row_tiles, hipStream_t stream) {
  if (p.K % 128 || p.N % Tile::kBN) return AFD_ERR_SHAPE;
  // resident workgroups per CU (registers and LDS decide); initialized once, thread-safely
  static const int per_cu = [] {
    int b = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, fp8_gemm_kernel<MODE>, Tile::kThreads, 0) !=
            hipSuccess ||
        b < 1)
      b = 1;
    return b;
  }();
  const int max_tiles = max_row_tiles * (p.N / Tile::kBN);
  int grid = device_cu_count() * per_cu;
  if (max_tiles < grid) grid = max_tiles < 1 ? 1 : max_tiles;
  hipLaunchKernelGGL(fp8_gemm_kernel<MODE>, dim3(grid), dim3(Tile::kThreads), 0, stream, p);
  AFD_CHECK_LAUNCH();
  return AFD_OK;
}

static Fp8GemmArgs common_args(const afd_moe_cfg& cfg, uint8_t* ws, const afd_ws_layout& L) {
  Fp8GemmArgs p = {};
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

}  // namespace fp8

int launch_fp8_gate_up(const afd_moe_cfg& cfg, const afd_expert_weights& wt, uint8_t* ws,
                       const afd_ws_layout& L, const uint8_t* xq, const void* xs,
                       const afd_job* rows_desc, hipStream_t stream) {
  fp8::Fp8GemmArgs p = fp8::common_args(cfg, ws, L);
  p.a = xq;
  p.as = static_cast<const float*>(xs);
  p.rows_desc = rows_desc;
  p.b = static_cast<const uint8_t*>(wt.w13);
  p.bs = static_cast<const float*>(wt.s13);
  p.walk_ctr = cfg.tile_walk == AFD_WALK_DYNAMIC ? call_counters(ws, L) + kGateUpWalkWord : nullptr;
  p.K = cfg.hidden;
  p.N = 2 * cfg.inter;
  p.hq = ws + L.hq;
  p.hs = reinterpret_cast<float*>(ws + L.hs);
  return cfg.activation != AFD_ACT_SWIGLU ? fp8::launch<fp8::kGateUpParam>(p, L.max_tiles, stream)
                                         : fp8::launch<fp8::kGateUp>(p, L.max_tiles, stream);
}

int launch_fp8_down(const afd_moe_cfg& cfg, const afd_expert_weights& wt, uint8_t* ws,
                    const afd_ws_layout& L, int32_t n, hipStream_t stream) {
  (void)n;
  fp8::Fp8GemmArgs p = fp8::common_args(cfg, ws, L);
  p.a = ws + L.hq;
  p.as = reinterpret_cast<const float*>(ws + L.hs);
  p.b = static_cast<const uint8_t*>(wt.w2);
  p.bs = static_cast<const float*>(wt.s2);
  p.walk_ctr = cfg.tile_walk == AFD_WALK_DYNAMIC ? call_counters(ws, L) + kDownWalkWord : nullptr;
  p.K = cfg.inter;
  p.N = cfg.hidden;
  p.y = reinterpret_cast<uint16_t*>(ws + L.y);
  return fp8::launch<fp8::kDown>(p, L.max_tiles, stream);
}

}  // namespace afd
