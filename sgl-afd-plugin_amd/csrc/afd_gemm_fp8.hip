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
  uint32_t* walk_ctr;             // zeroed tile counters, XCD x's at x * kWalkCounterStride; nullptr: static walk
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
  // down: a ring of 4 such stages (one more stage in flight than 3 measured 3% faster), its
  // epilogue's bf16 tile over the ring
  static constexpr int kStages = 4;
  static constexpr int kYBytes = kBM * kBN * 2;
  static constexpr int kDownLds = kStages * kStage > kYBytes ? kStages * kStage : kYBytes;
  // per wavefront and stage: 2 pieces of the A block and 2 of the weight image; wavefronts
  // 0-3 also copy the scale words of rows [64 w, 64 w + 64)
  static constexpr int kAQ = (kImgF8B / 1024) / kWaves;
  static constexpr int kQP = (kImgF8B / 1024) / kWaves;
  static constexpr int kPiecesMin = kAQ + kQP;  // pieces of a wavefront without scales
  static constexpr int kYChunks = kBN / 8;
  // gate_up gathers its A rows from the token rows, whose 64-byte halves a 64-K stage would
  // take as two requests of the same 128-byte line; it copies them per 128-K superstage
  // instead: an A ring of 2 superstages (256 rows x 128 B, in the MXFP8 A image's layout,
  // img_a_off), a ring of 3 weight images, the per-stage scale slots of the fallback (see the
  // kernel), the epilogue's per-row amax of each column wavefront [2][256 rows], and the
  // scale table (K up to 4096)
  static constexpr int kGASlot = kBM * 128;
  static constexpr int kGB = 2 * kGASlot;
  static constexpr int kGS = kGB + 3 * kImgF8B;
  static constexpr int kGAmax = kGS + 3 * kBM * 4;
  static constexpr int kGTab = kGAmax + 2 * kBM * 4;
  static constexpr int kTabMaxChunks = 8;  // 16-byte chunks (4 K blocks) per row: K <= 4096
  static constexpr int kGateUpLds = kGTab + kTabMaxChunks * kBM * 16;
  static constexpr int kGAQ = (kGASlot / 1024) / kWaves;  // A pieces of a wavefront and superstage
  static_assert(kBM == 256 && kAQ * kWaves * 1024 == kImgF8B && kGAQ * kWaves * 1024 == kGASlot,
                "pieces cover a stage");
  static_assert((kStage & 255) == 0 && (kGB & 255) == 0,
                "slot offsets leave the fragment addresses' low 8 bits alone");
  static_assert(kDownLds + 256 <= 160 * 1024 && kGateUpLds + 256 <= 160 * 1024, "LDS of one CU");
  template <int MODE>
  static constexpr int lds_bytes() { return MODE == 1 ? kDownLds : kGateUpLds; }
  static_assert(4 * (kPiecesMin + 1) < 64 && kQP + 2 * (kGAQ + kQP) + 1 < 64, "vmcnt is a 6-bit counter");
};

// A uniform read of data the kernel never writes (the weight block scales), through the
// scalar cache: a vector load's wait would drain the copies in flight.
__device__ __forceinline__ float load_uniform(const float* p) {
  return *(const __attribute__((address_space(4))) float*)p;
}

template <int MODE>
__global__ __launch_bounds__(Tile::kThreads) void fp8_gemm_kernel(Fp8GemmArgs p) {
  using T = Tile;
  constexpr int kBM = T::kBM, kBN = T::kBN, kStages = T::kStages, kStage = T::kStage;
  constexpr bool kGU = MODE != kDown;
  constexpr int kNA = kGU ? T::kGAQ : T::kAQ;  // A pieces of a wavefront per (super)stage
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
  // fragment bases of the lane: weight row 128 wn + lr at logical chunk lk (the operand's
  // first 16 bytes; its second 16 are logical chunk lk + 2, i.e. the address with bit 5
  // flipped), A row 64 wm + lr the same way (down) or (gate_up, 128-byte rows) the row's
  // swizzled base, XORed with the chunk per read. Rows + 32 i keep the 64-byte rows' swizzle
  // and flip chunk bit 2 of the 128-byte rows'.
  const int a_lane = kGU ? 0 : img_b_off(wm * 64 + lr, lk);
  int a_ch[4] = {};  // gate_up: chunks lk, lk + 2, lk + 4, lk + 6 of the lane's A row
  if constexpr (kGU) {
#pragma unroll
    for (int j = 0; j < 4; ++j) a_ch[j] = img_a_off(wm * 64 + lr, lk + 2 * j);
  }
  const int b_lane = (kGU ? T::kGB : T::kBOff) + img_b_off(wn * 128 + lr, lk);
  // gate_up's activation-row scales: with K a multiple of 512 up to 4096, every row's K-block
  // scales (K / 128 words, contiguous in xs) are copied once per tile into the scale table;
  // otherwise wavefronts 0-3 copy the 256 rows' words of each stage's K block into its slot.
  // The table holds 16-byte chunk c (the scales of K blocks 4 c .. 4 c + 3) of row r at
  // (256 c + r) * 16 (a read of one block's scale of 32 rows: two-way bank conflicts, once
  // per 128 K); wavefront w copies chunks c = 2 q + w / 4 of rows 64 (w % 4) + lane.
  const int tab_chunks = kb_n / 4;
  const bool table = kGU && kb_n % 4 == 0 && tab_chunks <= T::kTabMaxChunks;
  const bool copies_scales = w_u < 4 && !table;
  auto tab_off = [&](int r, int c) { return T::kGTab + (c * kBM + r) * 16; };

  // Tile metadata one tile ahead (as the W4A8 kernel). gate_up gathers its A superstages from
  // the token rows: lane l copies, for its piece q (8 rows of 128 B), physical chunk l % 8 of
  // row 8 (w kGAQ + q) + l / 8, i.e. logical chunk (l % 8) ^ swizzle(row), from the row's
  // token; the scale words (fallback) and the table chunks of wavefront w are those of row
  // 64 (w % 4) + l. Padding rows (-1) read token 0; their results are never stored.
  int sp_next[kNA + 1], e_next = 0, own_next = -1;
  auto load_next = [&](int ii) {
    int m, nn;
    walk.at_dense(ii, m, nn);
    e_next = p.tile_expert[m];
    own_next = p.sorted_pairs[m * kBM + 64 * wm + lane];
    if constexpr (MODE != kDown) {
#pragma unroll
      for (int q = 0; q < kNA; ++q)
        sp_next[q] = p.sorted_pairs[m * kBM + 8 * (w_u * kNA + q) + (lane >> 3)];
      sp_next[kNA] = p.sorted_pairs[m * kBM + 64 * (w_u & 3) + lane];
    }
  };
  int e_cur = 0, live_cur = 0;
  uint32_t a_voff[kNA] = {}, s_voff = 0;
  auto decode_next = [&]() {
    e_cur = __builtin_amdgcn_readfirstlane(e_next);
    live_cur = __popcll(__ballot(own_next >= 0));  // real rows of this group, a scalar
    if constexpr (MODE != kDown) {
      auto token = [&](int sp) {
        return sp >= 0 ? div_by_magic(static_cast<uint32_t>(sp), p.topk_magic) : 0u;
      };
#pragma unroll
      for (int q = 0; q < kNA; ++q) {
        const int r = 8 * (w_u * kNA + q) + (lane >> 3);
        const int c = (img_a_off(r, lane & 7) - r * 128) >> 4;  // the swizzle is an involution
        a_voff[q] = token(sp_next[q]) * static_cast<uint32_t>(p.K) + c * 16;
      }
      s_voff = token(sp_next[kNA]) * static_cast<uint32_t>(kb_n * 4);
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
  // down: this wavefront's copies of stage kt into ring slot kt % 4: its A pieces, its weight
  // pieces, and (wavefronts 0-3) scale words
  auto issue_down = [&](int kt) {
    const uint32_t st = lds_base + static_cast<uint32_t>((kt % kStages) * kStage);
    static_for<T::kAQ>([&](auto qc) {
      constexpr int q = decltype(qc)::value;
      const int off = (w_u * T::kAQ + q) * 1024;
      lds_dma16(st + off, a_tile + int64_t(kt) * kImgF8B + off, voff);
    });
    static_for<T::kQP>([&](auto qc) {
      constexpr int q = decltype(qc)::value;
      const int off = (w_u * T::kQP + q) * 1024;
      lds_dma16(st + T::kBOff + off, b_tile + int64_t(kt) * kImgF8B + off, voff);
    });
    if (copies_scales)
      lds_dma4(st + T::kAScale + w_u * 256, s_tile + (kt >> 1) * kBM + 64 * w_u, lane * 4u);
  };
  // gate_up: its A pieces of superstage sk (K [128 sk, + 128)) into A slot sk % 2; its weight
  // pieces of stage kt into B slot kt % 3, with (fallback, wavefronts 0-3) the scale words
  auto issue_a = [&](int sk) {
    const uint32_t st = lds_base + static_cast<uint32_t>((sk & 1) * T::kGASlot);
    static_for<kNA>([&](auto qc) {
      constexpr int q = decltype(qc)::value;
      lds_dma16(st + (w_u * kNA + q) * 1024, a_tile + int64_t(sk) * 128, a_voff[q]);
    });
  };
  auto issue_b = [&](int kt) {
    const int slot = kt % 3;
    const uint32_t st = lds_base + static_cast<uint32_t>(T::kGB + slot * kImgF8B);
    static_for<T::kQP>([&](auto qc) {
      constexpr int q = decltype(qc)::value;
      const int off = (w_u * T::kQP + q) * 1024;
      lds_dma16(st + off, b_tile + int64_t(kt) * kImgF8B + off, voff);
    });
    if (copies_scales)
      lds_dma4(lds_base + static_cast<uint32_t>(T::kGS + slot * kBM * 4 + w_u * 256), s_tile + (kt >> 1), s_voff);
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
  const int last_sk = KT / 2 - 1;  // the last superstage (KT is even)
  // A tile's K loop starts with every ring slot filled, issued during the previous tile's
  // epilogue (gate_up) or at the start of the tile (down). down: stages 0-3. gate_up: the
  // tile's table pieces (so the wait for stage 0 covers them; the previous tile's K loop, the
  // table's only reader, has ended by then), then A superstage 0, weights of stages 0 and 1,
  // then what the loop itself would have issued at stage 0: A superstage 1 and weights of
  // stage 2 (all clamped to the last (super)stage: a clamped copy rewrites a slot with its
  // own bytes, and keeps every wavefront's count of copies in flight the same at each wait).
  auto issue_first = [&]() {
    if constexpr (kGU) {
      if (table) {
        for (int c = w_u >> 2; c < tab_chunks; c += 2)
          lds_dma16(lds_base + static_cast<uint32_t>(tab_off(64 * (w_u & 3), c)), s_tile,
                    s_voff + static_cast<uint32_t>(c * 16));
      }
      issue_a(0);
      issue_b(0);
      issue_b(min(1, last));
      issue_a(min(1, last_sk));
      issue_b(min(2, last));
    } else {
      static_for<kStages>([&](auto sc) { issue_down(min(static_cast<int>(decltype(sc)::value), last)); });
    }
  };
  // the copies issued at stage kt >= 1 of the K loop: gate_up A superstage kt / 2 + 1 (at even
  // kt) and weights of stage kt + 2; down stage kt + 3
  auto issue = [&](int kt) {
    if constexpr (kGU) {
      if ((kt & 1) == 0) issue_a(min(kt / 2 + 1, last_sk));
      issue_b(min(kt + 2, last));
    } else {
      issue_down(min(kt + kStages - 1, last));
    }
  };
  // Copies complete in issue order, so each wait leaves in flight exactly what was issued
  // after the last piece the next stage needs (a wavefront that also copies scale words waits
  // for a piece or two more than it needs): down, one stage of copies; gate_up, at the end of
  // an even stage (the next stage needs only its weights) the copies issued at this stage, at
  // the end of an odd stage (the next needs A superstage and weights issued at the stage
  // before) the weights issued at this stage. Before stage 0: everything after stage 0's
  // weights.
  constexpr int kWaitFirst = kGU ? T::kQP + kNA + T::kQP : (kStages - 1) * T::kPiecesMin;
  constexpr int kWaitEven = kGU ? kNA + T::kQP : (kStages - 2) * T::kPiecesMin;
  constexpr int kWaitOdd = kGU ? T::kQP : (kStages - 2) * T::kPiecesMin;
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
    // ks: the stage's k-step within its gate_up superstage (kt & 1)
    auto read_stage = [&](int kt, auto ks_c) {
      constexpr int ks = decltype(ks_c)::value;
      const int b0 = (kGU ? (kt % 3) * kImgF8B : (kt % kStages) * kStage) + b_lane;
      if constexpr (kGU) {
        // row r0 + 32 i2's chunk c sits 4096 B after row r0's chunk c ^ 4, so the four lane
        // addresses of chunks lk + 2 j serve both row blocks of both k-steps
        const uint8_t* as = lds + ((kt >> 1) & 1) * T::kGASlot;
#pragma unroll
        for (int i2 = 0; i2 < 2; ++i2) {
          const int j = 2 * (ks ^ i2);  // chunk lk + 2 j: the k-step's first 16 bytes
          const v4i lo = *reinterpret_cast<const v4i*>(as + a_ch[j] + 4096 * i2);
          const v4i hi = *reinterpret_cast<const v4i*>(as + a_ch[j + 1] + 4096 * i2);
          fa[i2] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
      } else {
        const int a0 = (kt % kStages) * kStage + a_lane;
#pragma unroll
        for (int i2 = 0; i2 < 2; ++i2) {
          const v4i lo = *reinterpret_cast<const v4i*>(lds + a0 + 2048 * i2);
          const v4i hi = *reinterpret_cast<const v4i*>(lds + (a0 ^ 32) + 2048 * i2);
          fa[i2] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
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
    int kb_next = 0;  // the K block whose weight scales swn0, swn1 hold
    auto block_scales = [&](int kt) {
      float x0, x1;
      if (MODE != kDown && table) {
        const int kb = kt >> 1;
        x0 = *reinterpret_cast<const float*>(lds + tab_off(wm * 64 + lr, kb >> 2) + (kb & 3) * 4);
        x1 = *reinterpret_cast<const float*>(lds + tab_off(wm * 64 + 32 + lr, kb >> 2) + (kb & 3) * 4);
      } else {
        const float* sxs = reinterpret_cast<const float*>(
            lds + (kGU ? T::kGS + (kt % 3) * kBM * 4 : (kt % kStages) * kStage + T::kAScale));
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
    wait_vmcnt<kWaitFirst>();  // own pieces of stage 0 landed
    __syncthreads();
    // The loops take two stages per iteration (KT is even), the K block's first with the
    // accumulators' factor and its second without, so neither MFMA phase branches on it (the
    // factor of block 0 multiplies zeros).
    if (w_u < 4) {
      auto phase = [&](int kt, auto first_c) {
        constexpr bool kFirst = decltype(first_c)::value;
        // the claim rides on the last stage, whose end waits for every copy anyway
        if (!kFirst && claims && kt == last) ticket = walk.claim_ticket();
        if (kt >= 1) issue(kt);
        read_stage(kt, std::integral_constant<int, kFirst ? 0 : 1>{});
        if constexpr (kFirst) block_scales(kt);
        wait_lds();  // own reads done (copies may be in flight)
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(1);
        mma_stage(kFirst);
        __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt<kFirst ? kWaitEven : kWaitOdd>();  // own pieces of stage kt + 1
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
        if (kt >= 1) issue(kt);
        read_stage(kt, std::integral_constant<int, kFirst ? 0 : 1>{});
        if constexpr (kFirst) block_scales(kt);
        wait_vmcnt_lds<kFirst ? kWaitEven : kWaitOdd>();  // own reads, own pieces of stage kt + 1
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
      float* amax_l = reinterpret_cast<float*>(lds + T::kGAmax);
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
          const float rsc = 1.0f / sc;  // the quotients below are the IEEE h / sc (div_by)
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) {
            uint32_t d[4];
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4)
              d[q4] = pk4_e4m3_near(div_by(h[i2][jj][4 * q4], sc, rsc), div_by(h[i2][jj][4 * q4 + 1], sc, rsc),
                               div_by(h[i2][jj][4 * q4 + 2], sc, rsc), div_by(h[i2][jj][4 * q4 + 3], sc, rsc));
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
