// Grouped MXFP4-weight x MXFP8-activation GEMMs of the expert FFN on gfx950 scaled MFMA
// (v_mfma_scale_f32_32x32x64_f8f6f4: A e4m3, B e2m1, one UE8M0 scale per lane = per 32 K).
//
//   gate_up: h[p, :] = silu(x_t . Wg_e^T) * (x_t . Wu_e^T) for every padded row p of expert e
//            (t = token of the pair at row p), quantized to MXFP8 in the epilogue and written
//            as the down GEMM's A operand images.
//   down:    y[p, :] = bf16(h_p . W2_e^T).
//
// Tiling: a workgroup of 2 x WN wavefronts owns a 128 x (128 WN) output tile; wavefront
// (wm, wn) owns 64 x 128 = 2 x 4 MFMA tiles of 32x32 (128 fp32 accumulators per lane).
// WN = 4 (8 wavefronts, two per SIMD, so one wavefront's LDS reads overlap the other's
// MFMAs) is used whenever N is a multiple of 512; WN = 2 otherwise. K advances 128 per stage
// (two MFMA k-steps). Both operands are stored as tile images (the LDS bytes of one stage,
// scales included: afd_common.h), so a stage is one A block of 16.5 KiB and WN/2 B blocks of
// 17 KiB that move HBM -> LDS with gfx950's direct global_load_lds in 1 KiB pieces, without
// register staging, into a ring of 3 stages.
//
// The workgroups are persistent: grid = resident workgroups, and the number of row tiles is
// read from device memory (the router wrote it), so no host round trip is needed. They walk
// the tiles XCD by XCD in blocks of 2 row tiles x 16 column tiles (TileWalk), so the
// workgroups of an XCD share activation rows and weight slices in their L2.
#include <type_traits>

#include "afd_common.h"
#include "afd_internal.h"

namespace afd {

// gate_up with SwiGLU, gate_up with an activation that takes constants (SiTU, or SwiGLU with
// a limit: SiTU's longer epilogue would raise the register pressure of the SwiGLU kernel),
// down
enum { kGateUp = 0, kDown = 1, kGateUpParam = 2 };

// Tile walk blocks of 2 row tiles x 16 column tiles (all 8 of a 4096-wide GEMM): a row tile's
// gathered activation rows are shared by all its column tiles, each XCD's 32 workgroups run
// 2 such blocks at a time (measured ~1% faster than 4 x 8 blocks on the DeepSeek-V4 F-rank
// layer, the job stream and the loop even; 8 x 4 blocks, whose lower HBM traffic does not
// pay, no faster than 4 x 8).
constexpr int kMxWalkRows = 2;

struct MxGemmArgs {
  const uint8_t* a_img;         // down: A images [row tiles][K/128]
  const uint8_t* a_rows;        // gate_up: e4m3 token rows [n][K], gathered by sorted_pairs
  const uint8_t* a_scales;      // gate_up: their UE8M0 scales [n][K/32] in stage order
  const afd_job* rows_desc;     // gate_up: if set, a_rows / a_scales are its xq / xs
  int topk;                     // gate_up: pairs per token (token of pair p = p / topk)
  uint32_t topk_magic;          // div_magic(topk)
  const uint8_t* b_img;         // B images [E][N/256][K/128]
  const int32_t* sorted_pairs;  // [np] flat pair index per padded row, -1 = pad
  const int32_t* tile_expert;   // [row tiles]
  const int32_t* num_tiles;     // [1]
  const int32_t* padded_offsets;  // [E + 1] first padded row of each expert
  const int32_t* counts;          // [E] pairs of each expert (its first rows)
  uint32_t* walk_ctr;             // zeroed tile counters, XCD x's at x * kWalkCounterStride; nullptr: static walk
  int K, N;
  uint8_t* h_img;  // gate_up out: the down GEMM's A images [row tiles][N/256]
  ActParams act;   // gate_up: the activation
  uint16_t* y;     // down out: bf16 [np][N]
};

// Shape of the workgroup tile: 2 x WN wavefronts in two groups of WN (group g = rows
// [64 g, 64 g + 64)), BN = 128 WN columns.
template <int WN>
struct MxTile {
  static_assert(WN == 2 || WN == 4, "tiles are 256 or 512 columns wide");
  static constexpr int kWaves = 2 * WN;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kBM = kBlockM;  // 128 rows = one A image
  static constexpr int kBN = 128 * WN;
  static constexpr int kBImgs = WN / 2;  // 256-row B images per tile
  // LDS stage: the A image (its 512 B of scales padded to a 1 KiB piece), then the B images
  static constexpr int kLdsA = kImgData + 1024;
  static constexpr int kStage = kLdsA + kBImgs * kImgB;
  static constexpr int kStages = 3;
  static constexpr int kLds = kStages * kStage;
  // a stage is kImgs images of 17 pieces of 1 KiB: every wavefront copies kQP of the 16 data
  // pieces of each image plus one scale piece (scale pieces past the real ones repeat one:
  // the same bytes to the same place)
  static constexpr int kImgs = 1 + kBImgs;
  static constexpr int kQP = 16 / kWaves;
  static constexpr int kPieces = kImgs * kQP + 1;
  static_assert(kWaves >= 2 * kImgs, "a scale piece per image, two for a gathered A");
  // the down epilogue's bf16 tile: kBM rows of kBN / 8 16-byte chunks, chunk c of row r at
  // physical chunk c ^ (r % 16), so the 16 rows a 16-lane pass of a write covers (one logical
  // chunk each) and the 16 consecutive chunks a pass of a read covers (one row) fall on 16
  // distinct 16-byte bank groups
  static constexpr int kYChunks = kBN / 8;
  static_assert(kBM * kBN * 2 <= kLds, "down epilogue tile must fit the stages");
  static_assert(kImgB == 17 * 1024, "B images are 17 pieces of 1 KiB");
  static_assert(kLds <= 160 * 1024, "LDS of one CU");
  static_assert(2 * kPieces < 64, "vmcnt is a 6-bit counter");
};

// The scaled MFMA with a 4-dword (e2m1) B operand. The clang builtin takes 8 dwords for every
// operand format; the intrinsic's B operand type follows the format, and e2m1 needs only 4.
// The kernels pass the e2m1 weights as the first operand and the e4m3 activations as the
// second (D = W X^T), so a lane's accumulators belong to one activation row.
extern "C" __device__ v16f mfma_scale_f4_f8(v4i a, v8i b, v16f c, int cbsz, int blgp,
                                            int opsel_a, int scale_a, int opsel_b, int scale_b)
    __asm("llvm.amdgcn.mfma.scale.f32.32x32x64.f8f6f4.v4i32.v8i32");

// kCont false: each tile fills the ring, runs its K loop, drains the ring and runs its
// epilogue. kCont (gate_up with at least 3 K stages, static walk): the copy ring runs on across
// tiles (the next tile's first stages are copied during the current tile's last two, like any
// other stage) and each group's epilogue runs in its next read phase, beside the other group's
// MFMAs. The dynamic walk keeps the first form: its claim's result would be a counted load
// that the compiler waits for (draining the ring) wherever that register is copied or reused,
// while the first form claims during a last stage whose end waits for every copy anyway.
template <int MODE, int WN, bool kCont>
__global__ __launch_bounds__(MxTile<WN>::kThreads) void mx_gemm_kernel(MxGemmArgs p) {
  static_assert(!kCont || MODE != kDown, "the continuous ring is gate_up's (down stages y in LDS)");
  using T = MxTile<WN>;
  constexpr int kBM = T::kBM, kBN = T::kBN, kStages = T::kStages, kStage = T::kStage;
  __shared__ __attribute__((aligned(16))) uint8_t lds[T::kLds];
  const int t = threadIdx.x, lane = t & 63;
  const int w_u = __builtin_amdgcn_readfirstlane(t >> 6);  // wavefront index, scalar
  const int wm = w_u / WN, wn = w_u % WN, lr = lane & 31, lk = lane >> 5;
  const int nt256 = p.N / kImgBRows;
  const TileWalk<kMxWalkRows> walk(p.num_tiles[0], p.N / kBN, blockIdx.x, gridDim.x, p.walk_ctr);
  // lane 0 claims the walk's dense positions (the tile after next, one tile ahead) and
  // publishes them here; every wavefront reads them after a barrier
  __shared__ int claimed[2];
  // continuous ring: the next row tile's 128 pair indices, then its expert (64 copies)
  __shared__ __attribute__((aligned(16))) int32_t meta[kCont ? kBM + 64 : 1];
  // vector-memory instructions of one wavefront's gate_up epilogue: a 16-byte h chunk and a
  // scale byte per MX block (2 x 2 blocks)
  constexpr int kEpiStores = 8;
  const int KT = p.K / kImgK;
  const uint32_t lds_base = __builtin_amdgcn_readfirstlane(lds_offset(lds));
  const uint32_t voff = static_cast<uint32_t>(lane) * 16;
  const uint8_t* a_rows = p.a_rows;
  const uint8_t* a_scales = p.a_scales;
  if (MODE != kDown && p.rows_desc != nullptr) {
    a_rows = p.rows_desc->xq;
    a_scales = static_cast<const uint8_t*>(p.rows_desc->xs);
  }
  // this wavefront's B operand: image wn/2 of the stage, rows (wn%2)*128 + j*32 + lr
  const int bimg = wn / 2, brow = (wn % 2) * 128;

  // A tile's metadata is loaded one tile ahead and decoded after the previous tile's K loop,
  // whose last wait leaves no copy in flight, so no tile starts by waiting for a load.
  // gate_up gathers its A operand from the token rows: a lane copies one 16-byte chunk of row
  // 8 (w kQP + q) + lane / 8 of the tile for each of its A pieces q (physical chunk lane % 8,
  // so logical chunk (lane % 8) ^ swizzle(row)) and the scale word of row 64 h + lane for
  // scale half h, at offsets given by the pair indices of those rows. Padding rows (-1) read
  // token 0; their results are never stored.
  const int s_half = (w_u / T::kImgs) & 1;
  // Each wavefront also loads the pair indices of its group's 64 rows: an expert's padding
  // rows (-1) come last in its segment, so a ballot counts the group's real rows, and MFMAs
  // of 32-row blocks with no real row are skipped (their rows are never stored).
  int sp_next[T::kQP + 1], e_next = 0, own_next = -1;
  auto load_next = [&](int ii) {
    int m, nn;
    walk.at_dense(ii, m, nn);
    e_next = p.tile_expert[m];
    own_next = p.sorted_pairs[m * kBM + 64 * wm + lane];
    if constexpr (MODE != kDown) {
#pragma unroll
      for (int q = 0; q < T::kQP; ++q)
        sp_next[q] = p.sorted_pairs[m * kBM + 8 * (w_u * T::kQP + q) + (lane >> 3)];
      sp_next[T::kQP] = p.sorted_pairs[m * kBM + 64 * s_half + lane];
    }
  };
  int e_cur = 0, live_cur = 0;
  uint32_t a_voff[T::kQP] = {}, s_voff = 0;
  auto decode_next = [&]() {
    e_cur = __builtin_amdgcn_readfirstlane(e_next);
    live_cur = __popcll(__ballot(own_next >= 0));  // real rows of this group, a scalar
    if constexpr (MODE != kDown) {
      auto token = [&](int sp) {
        return sp >= 0 ? div_by_magic(static_cast<uint32_t>(sp), p.topk_magic) : 0u;
      };
#pragma unroll
      for (int q = 0; q < T::kQP; ++q) {
        const int r = 8 * (w_u * T::kQP + q) + (lane >> 3);
        const int c = (lane & 7) ^ ((r ^ (r >> 3)) & 7);
        a_voff[q] = token(sp_next[q]) * p.K + c * 16;
      }
      s_voff = token(sp_next[T::kQP]) * (p.K / 32);
    }
  };
  // The tile whose stages the copies below fetch. gate_up issues the next tile's first two
  // stages right after its own K loop: its epilogue works from registers, so those copies
  // land while it runs. down's epilogue stages its output through the LDS ring, so it issues
  // them at the start of the tile.
  constexpr bool kEarlyStart = MODE != kDown;
  const uint8_t* a_tile = nullptr;
  const uint8_t* b_tile = nullptr;
  const uint8_t* src16 = nullptr;
  // this wavefront's copies of stage kt into ring slot kt % 3: piece c of image c / 17 (0 = A,
  // its 17th piece being the scales plus the 512 B that follow them in memory). Scalar
  // address arithmetic only, so the issuing code has no branches.
  // Piece q of this wavefront: for q < kImgs * kQP, piece w * kQP + q % kQP of image
  // q / kQP (0 = A, then the B images). The last, q = kImgs * kQP, is a scale piece:
  // wavefront w < 2 kImgs copies that of image w % kImgs (of the gathered A of gate_up, half
  // w / kImgs: 64 rows' words), later wavefronts repeat a B image's (the same bytes to the
  // same place), so the costly gathered scale copy is issued once per half. Only the last
  // piece depends on the wavefront beyond an offset, so it is resolved once per tile; the
  // others are address arithmetic.
  const int img16 = w_u < 2 * T::kImgs ? w_u % T::kImgs : 1 + (w_u - 2 * T::kImgs) % T::kBImgs;
  const int step16 = img16 == 0 ? kImgA : kImgB;
  const uint32_t dst16 = img16 == 0 ? kImgData : T::kLdsA + (img16 - 1) * kImgB + kImgData;
  auto copy_tile = [&](int mt, int nt, int64_t e) {
    a_tile = MODE == kDown ? p.a_img + int64_t(mt) * KT * kImgA : a_rows;
    b_tile = p.b_img + (e * nt256 + int64_t(nt) * T::kBImgs) * KT * int64_t(kImgB);
    src16 = img16 == 0 ? a_tile + kImgData : b_tile + int64_t(img16 - 1) * KT * kImgB + kImgData;
  };
  auto issue_piece = [&](int kt, uint32_t slot_off, auto qc) {
    constexpr int q = decltype(qc)::value;
    const uint32_t st = lds_base + slot_off;
    if constexpr (q == T::kImgs * T::kQP) {
      if (MODE != kDown && img16 == 0)  // 64 rows' scale words, gathered
        lds_dma4(st + kImgData + s_half * 256, a_scales + int64_t(kt) * 4, s_voff);
      else
        lds_dma16(st + dst16, src16 + int64_t(kt) * step16, voff);
    } else {
      constexpr int img = q / T::kQP;
      const int off = (w_u * T::kQP + q % T::kQP) * 1024;
      if constexpr (img == 0 && MODE != kDown)
        lds_dma16(st + off, a_rows + int64_t(kt) * kImgK, a_voff[q % T::kQP]);
      else if constexpr (img == 0)
        lds_dma16(st + off, a_tile + int64_t(kt) * kImgA + off, voff);
      else
        lds_dma16(st + T::kLdsA + (img - 1) * kImgB + off,
                  b_tile + (int64_t(img - 1) * KT + kt) * kImgB + off, voff);
    }
  };
  // stage kt of the copy tile into the ring slot at byte offset slot_off
  auto issue_at = [&](int kt, uint32_t slot_off) {
    static_for<T::kPieces>([&](auto q) { issue_piece(kt, slot_off, q); });
  };
  auto issue = [&](int kt) { issue_at(kt, static_cast<uint32_t>((kt % kStages) * kStage)); };
  const int last = KT - 1;

  // The walk's dense positions: static (this workgroup's first, first + stride, ...) or,
  // with p.walk_ctr, claimed one tile ahead by lane 0 from its XCD's counter (the first two
  // here, each later one during the last K stage of the tile before the one that needs it).
  const bool dynamic = !kCont && p.walk_ctr != nullptr;
  int i = walk.first, i_next = walk.first + walk.stride;
  if (dynamic) {
    if (t == 0) {
      // two increments in flight together (b > a, so b is past the last tile if a is)
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
  // (`ticket` lives across the tile loop, so no write to its register waits for the
  // increment; an increment, which the compiler's atomic combining leaves alone, so nothing
  // waits for its result before the use)
  uint32_t ticket = 0;

  v16f acc[2][4];
  auto zero_acc = [&]() {
#pragma unroll
    for (int i2 = 0; i2 < 2; ++i2)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int q = 0; q < 16; ++q) acc[i2][j][q] = 0.0f;
  };
  // 32-row blocks i of this group with a real row, in the tile being multiplied
  bool live_i0 = false, live_i1 = false;

  // Operand fragments of both k-steps of one stage, with the stage's scale words.
  // 8-bit operand of the f8f6f4 MFMA: lane half h holds K [16h, 16h+16) in bytes 0-15 and
  // K [32+16h, 32+16h+16) in bytes 16-31 of the k-step; the e2m1 operand holds K [32h, 32h+32);
  // the scale of lane x+32b covers K block b.
  struct Frag {
    v8i a[2][2];  // [ks][i]
    v4i b[2][4];  // [ks][j]
    uint32_t sa[2], sb[4];  // bytes 0, 1: the scales of k-steps 0, 1 for this lane half
  };
  Frag f;
  auto read_stage = [&](int s) {
    const uint8_t* abase = lds + s * kStage;
    const uint8_t* bbase = abase + T::kLdsA + bimg * kImgB;
    const uint16_t* sa = reinterpret_cast<const uint16_t*>(abase + kImgData) + lk;
    const uint16_t* sb = reinterpret_cast<const uint16_t*>(bbase + kImgData) + lk;
    // Row r + 32 has the swizzle of row r with chunk bit 2 flipped, so its chunk c sits 4096 B
    // after row r's chunk c ^ 4: four lane addresses serve both row blocks, the second through
    // the instruction's offset field.
    const int r0 = wm * 64 + lr;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int i2 = 0; i2 < 2; ++i2) {
        const int kc = (ks ^ i2) * 4 + lk;
        f.a[ks][i2].lo = *reinterpret_cast<const v4i*>(abase + img_a_off(r0, kc) + i2 * 4096);
        f.a[ks][i2].hi = *reinterpret_cast<const v4i*>(abase + img_a_off(r0, kc + 2) + i2 * 4096);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
        f.b[ks][j] = *reinterpret_cast<const v4i*>(bbase + img_b_off(brow + j * 32 + lr, ks * 2 + lk));
    }
#pragma unroll
    for (int i2 = 0; i2 < 2; ++i2) f.sa[i2] = sa[2 * (wm * 64 + i2 * 32 + lr)];
#pragma unroll
    for (int j = 0; j < 4; ++j) f.sb[j] = sb[2 * (brow + j * 32 + lr)];
  };
  // the 16 MFMAs of a stage (blocks of padding rows skipped)
  auto mma_stage = [&]() {
    static_for<2>([&](auto ksc) {
      constexpr int ks = decltype(ksc)::value;
      static_for<2>([&](auto i2c) {
        constexpr int i2 = decltype(i2c)::value;
        static_for<4>([&](auto jc) {
          constexpr int j = decltype(jc)::value;
          // D[weight row][activation row]; op_sel ks: byte ks of the lane's scale half-word
          if (i2 == 0 ? live_i0 : live_i1)
            acc[i2][j] = mfma_scale_f4_f8(f.b[ks][j], f.a[ks][i2], acc[i2][j], 4 /*A e2m1*/,
                                          0 /*B e4m3*/, ks, static_cast<int>(f.sb[j]), ks,
                                          static_cast<int>(f.sa[i2]));
        });
      });
    });
  };

  // gate_up epilogue of row tile mt, columns [n0, n0 + kBN), from the accumulators.
  // Accumulator q of tile (i, j): activation row 64 wm + 32 i + lane % 32, output column
  // 128 wn + 32 j + 8 (q / 4) + 4 (lane / 32) + q % 4. Column tiles j = 2 jj and 2 jj + 1 are
  // the gate and up halves of one 64-row group of interleaved W13, i.e. the same 32
  // intermediate columns: one MX block of h per (i, jj), 16 values in this lane and 16 in
  // lane ^ 32. The block's scale needs one exchange; then lane half lk assembles 16-byte chunk
  // lk of the block (h columns 16 lk .. 16 lk + 15) with a second, and stores it into the down
  // GEMM's A image (stage n0 / 256 + block / 4 of row tile mt). Exactly kEpiStores
  // vector-memory instructions per wavefront (inline assembly, so the count is fixed): the
  // continuous ring's waits count them.
  auto gate_up_epilogue = [&](int mt, int n0) __attribute__((always_inline)) {
    const int kt_down = p.N / kImgBRows;  // K stages of the down GEMM (I / 128)
    // lane-derived addresses are computed here, not kept live through the K loop
    const int ln = opaque(lane), lr = ln & 31, lk = ln >> 5;
    auto quant_store = [&](auto fn) {
      static_for<2>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        static_for<2>([&](auto jjc) {
          constexpr int jj = decltype(jjc)::value;
          float h[16];
          float amax = 0.0f;
#pragma unroll
          for (int q = 0; q < 16; ++q) {
            h[q] = fn(acc[i][2 * jj][q], acc[i][2 * jj + 1][q]);
            amax = fmaxf(amax, fabsf(h[q]));
          }
          amax = fmaxf(amax, xor32(amax, lk));
          const uint32_t code = mx_scale_code(amax, 8);
          const float inv = mx_inv_scale(code);
          uint32_t d[4];  // h columns 8 q4 + 4 lk .. + 3
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4)
            d[q4] = pk4_e4m3(h[4 * q4] * inv, h[4 * q4 + 1] * inv, h[4 * q4 + 2] * inv,
                             h[4 * q4 + 3] * inv);
          // lane half 0 takes columns 0-15 (its d0, d1 and the partner's), half 1 columns
          // 16-31 (the partner's d2, d3 and its own)
          const uint32_t p0 = swap_halves(d[2], d[0], lk);
          const uint32_t p1 = swap_halves(d[3], d[1], lk);
          v4i chunk;
          chunk[0] = static_cast<int>(lk ? p0 : d[0]);
          chunk[1] = static_cast<int>(lk ? d[2] : p0);
          chunk[2] = static_cast<int>(lk ? p1 : d[1]);
          chunk[3] = static_cast<int>(lk ? d[3] : p1);
          const int row = wm * 64 + i * 32 + lr;
          const int hblk = wn * 2 + jj;  // MX block among the tile's kBN / 64
          uint8_t* img = p.h_img + (int64_t(mt) * kt_down + n0 / kImgBRows + hblk / 4) * kImgA;
          const int jb = hblk % 4;
          store16(img + img_a_off(row, 2 * jb + lk), chunk);
          // both lane halves hold the block's code (the amax was exchanged): the same byte to
          // the same place
          store8(img + kImgData + row * 4 + scale_byte(jb), code);
        });
      });
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
  };

  if constexpr (kCont) {
    // Continuous ring. Stages are numbered across tiles and take ring slots in turn; a tile's
    // stage kt + 2 (past its last: the next tile's stage kt + 2 - KT, or a rewrite of the last
    // stage into the free slot if there is no next tile) is copied when stage kt is read, so
    // the copies never drain. The copies switch to the next tile two stages before the end: by
    // then its 128 pair indices and its expert, copied into `meta` by direct-to-LDS copies of
    // waves 0-2 at the tile's first stage (older than that stage's ring copies, so that
    // stage's waits cover them), are decoded from LDS. A group's epilogue of the previous tile
    // runs in its first read phase of the next tile, beside the other group's MFMAs; its
    // kEpiStores stores are issued after that stage's copies, so the waits of that stage
    // allow them in flight, and the next stage's waits take them in.
    if (i >= walk.tiles) return;
    load_next(i);
    decode_next();
    int mt, nt;
    walk.at_dense(i, mt, nt);
    copy_tile(mt, nt, e_cur);
    issue_at(0, 0);
    issue_at(1, kStage);
    wait_vmcnt<T::kPieces>();  // own pieces of stage 0 landed
    __syncthreads();
    if (wm != 0) __syncthreads();  // group 1 runs half a stage behind group 0
    const uint32_t meta_lds = lds_offset(meta);
    // the tile loop of one group (kG0: group 0), instantiated per group so that each loop body
    // holds one form of the stage
    auto run = [&](auto grp) __attribute__((always_inline)) {
      constexpr bool kG0 = decltype(grp)::value;
      int rs = 0;  // ring slot of the stage read next
      int mt_prev = 0, n0_prev = 0;
      for (bool first = true;; first = false) {
        walk.at_dense(i, mt, nt);
        const bool has_next = i_next < walk.tiles;
        int mt1 = 0, nt1 = 0;
        if (has_next) walk.at_dense(i_next, mt1, nt1);
        live_i0 = live_cur > 0;
        live_i1 = live_cur > 32;
        auto stage = [&](int kt, auto epi) __attribute__((always_inline)) {
          constexpr int kSt = decltype(epi)::value ? kEpiStores : 0;
          if (kt == 0) {
            if (has_next && w_u < 3) {
              const int32_t* src = w_u == 2 ? p.tile_expert + mt1
                                            : p.sorted_pairs + int64_t(mt1) * kBM + 64 * w_u;
              lds_dma4(meta_lds + w_u * 256, src, w_u == 2 ? 0u : static_cast<uint32_t>(lane) * 4);
            }
          }
          if (kt == last - 1 && has_next) {
            const int ln = opaque(lane);
            e_next = meta[kBM];
            own_next = meta[64 * wm + ln];
  #pragma unroll
            for (int q = 0; q < T::kQP; ++q) sp_next[q] = meta[8 * (w_u * T::kQP + q) + (ln >> 3)];
            sp_next[T::kQP] = meta[64 * s_half + ln];
            decode_next();
            copy_tile(mt1, nt1, e_cur);
          }
          const int ck = kt + 2 <= last ? kt + 2 : has_next ? kt + 2 - KT : last;
          issue_at(ck, static_cast<uint32_t>((rs == 0 ? 2 : rs - 1) * kStage));
          if constexpr (decltype(epi)::value) gate_up_epilogue(mt_prev, n0_prev);
          if (kt == 0) zero_acc();
          read_stage(rs);
          if constexpr (kG0) {
            wait_vmcnt_lds<2 * T::kPieces + kSt>();  // own reads done (copies may be in flight)
            __syncthreads();
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_setprio(1);
            mma_stage();
            __builtin_amdgcn_s_setprio(0);
            __builtin_amdgcn_sched_barrier(0);
            wait_vmcnt<T::kPieces + kSt>();  // own pieces of the next stage landed
            __syncthreads();
          } else {
            wait_vmcnt_lds<T::kPieces + kSt>();  // own reads done, own next pieces landed
            __syncthreads();
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_setprio(1);
            mma_stage();
            __builtin_amdgcn_s_setprio(0);
            __builtin_amdgcn_sched_barrier(0);
            __syncthreads();
          }
          rs = rs == 2 ? 0 : rs + 1;
        };
        if (first)
          stage(0, std::false_type{});
        else
          stage(0, std::true_type{});
        for (int kt = 1; kt < KT; ++kt) stage(kt, std::false_type{});
        mt_prev = mt;
        n0_prev = nt * kBN;
        if (!has_next) break;
        i = i_next;
        i_next = min(i_next + walk.stride, walk.tiles);
      }
      // the last tile's epilogue: group 0's beside group 1's last MFMAs, then group 1's
      gate_up_epilogue(mt_prev, n0_prev);
      if constexpr (kG0) __syncthreads();
    };
    if (wm == 0)
      run(std::true_type{});
    else
      run(std::false_type{});
  } else {
    if (i < walk.tiles) {
      load_next(i);
      decode_next();
      if constexpr (kEarlyStart) {
        int mt, nt;
        walk.at_dense(i, mt, nt);
        copy_tile(mt, nt, e_cur);
        issue(0);
        issue(min(1, last));
      }
    }
    for (int i_after = walk.tiles; i < walk.tiles; i = i_next, i_next = i_after) {
      int mt, nt;
      walk.at_dense(i, mt, nt);
      const bool has_next = i_next < walk.tiles;
      const bool claims = dynamic && t == 0 && has_next;  // publishes the tile after next
      const int m0 = mt * kBM, n0 = nt * kBN;
      const int64_t e = e_cur;
      // down: the expert's pairs fill its first rows, padding the rest; rows below row_end are
      // real (loaded now, used by the epilogue)
      int row_end = 0;
      if constexpr (MODE == kDown) row_end = p.padded_offsets[e] + p.counts[e];
      live_i0 = live_cur > 0;
      live_i1 = live_cur > 32;
      if (has_next) load_next(i_next);
      if constexpr (!kEarlyStart) copy_tile(mt, nt, e);
      zero_acc();

      // Ping-pong: the two wavefronts of a SIMD (one per group) alternate between reading a
      // stage's operands from LDS and running its 16 MFMAs, half a stage apart, so one of them
      // always feeds the MFMA pipe while the other's reads proceed. All wavefronts meet at a
      // barrier every half stage; group 1 starts one barrier late and group 0 ends one
      // barrier later, so both execute 2 KT + 1 barriers per tile. The CU's vector-memory path
      // takes ~64 B/clk, so the copies are split between the groups, which keeps each read
      // phase shorter than the other group's MFMA phase. Each group copies its pieces of stage
      // kt+2 when it starts reading stage kt (copies issued between MFMAs delay them); the target
      // slot's previous stage was read by both groups before the barrier that started the phase.
      // Copies are clamped to the last stage (a clamped copy rewrites a slot with its own
      // bytes). Both groups wait for their own pieces of stage kt+1 in the phase before the
      // barrier after which group 0 reads stage kt+1: group 0 after its MFMAs of stage kt,
      // group 1 after its reads of stage kt.
      // epilogue stores of the previous tile may still be in flight (with kEarlyStart they were
      // issued after this tile's first copies): they only make the counted waits stricter
      // (vmcnt counts stores too; loads complete in order among themselves), never early
      if constexpr (!kEarlyStart) {
        issue(0);
        issue(min(1, last));
      }
      wait_vmcnt<T::kPieces>();  // own pieces of stage 0 landed
      __syncthreads();
      if (wm == 0) {
        for (int kt = 0; kt < KT; ++kt) {
          // the claim rides on the last stage, whose end waits for every copy anyway
          if (claims && kt == last) ticket = walk.claim_ticket();
          issue(min(kt + 2, last));
          read_stage(kt % kStages);
          wait_vmcnt_lds<2 * T::kPieces>();  // own reads done (copies may be in flight)
          __syncthreads();
          __builtin_amdgcn_sched_barrier(0);
          __builtin_amdgcn_s_setprio(1);
          mma_stage();
          __builtin_amdgcn_s_setprio(0);
          __builtin_amdgcn_sched_barrier(0);
          wait_vmcnt<T::kPieces>();  // own pieces of stage kt+1 landed
          __syncthreads();
        }
        __syncthreads();
      } else {
        __syncthreads();
        for (int kt = 0; kt < KT; ++kt) {
          issue(min(kt + 2, last));
          read_stage(kt % kStages);
          wait_vmcnt_lds<T::kPieces>();  // own reads done, own pieces of stage kt+1 landed
          __syncthreads();
          __builtin_amdgcn_sched_barrier(0);
          __builtin_amdgcn_s_setprio(1);
          mma_stage();
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
          issue(0);
          issue(min(1, last));
        }
      }

      if constexpr (MODE != kDown) {
        gate_up_epilogue(mt, n0);
      } else {
        // bf16 rows through LDS, so the stores write whole rows (a lane holds one row and only
        // 16-byte pieces of it: stored directly, 32 rows x 32 B per store instruction, the
        // down GEMM ran 4% slower, and 34% with the next tile's copies issued ahead). Lane half lk
        // holds columns 8 q4 + 4 lk .. + 3 of each 32-column tile; one exchange with the other
        // lane half per pair of chunks gives lane half lk whole 16-byte chunks q4 = lk and
        // 2 + lk, written with one 16-byte LDS write each. Rows [0, nvalid) of this tile are
        // real. The stores are non-temporal: y (np x H bf16) is read once, by the finalize, and
        // does not fit in L2 anyway.
        const int nvalid = min(kBM, row_end - m0);
        auto y_chunk = [](int r, int c) { return (r * T::kYChunks + (c ^ (r & 15))) * 16; };
        static_for<2>([&](auto ic) {
          constexpr int i = decltype(ic)::value;
          const int row = wm * 64 + i * 32 + lr;
          static_for<4>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            uint32_t h[4][2];  // the lane's 4 columns of chunk q4, as two bf16 pairs
  #pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
              h[q4][0] = pk_bf16(acc[i][j][4 * q4], acc[i][j][4 * q4 + 1]);
              h[q4][1] = pk_bf16(acc[i][j][4 * q4 + 2], acc[i][j][4 * q4 + 3]);
            }
  #pragma unroll
            for (int pr = 0; pr < 2; ++pr) {  // chunks 2 pr (lane half 0) and 2 pr + 1 (half 1)
              // v_permlane32_swap trades the first operand of lanes 32-63 for the second operand
              // of lanes 0-31: afterwards lane half 0 holds its own columns of chunk 2 pr and its
              // partner's, lane half 1 its partner's columns of chunk 2 pr + 1 and its own, both
              // in column order, with no select
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
}

template <int MODE, int WN, bool kCont>
static int launch_mx(const MxGemmArgs& p, int max_row_tiles, hipStream_t stream) {
  using T = MxTile<WN>;
  // resident workgroups per CU (registers and LDS decide); initialized once, thread-safely
  static const int per_cu = [] {
    int b = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, mx_gemm_kernel<MODE, WN, kCont>, T::kThreads,
                                                     0) != hipSuccess ||
        b < 1)
      b = 1;
    return b;
  }();
  const int max_tiles = max_row_tiles * (p.N / T::kBN);
  MxGemmArgs a = p;
  int grid = device_cu_count() * per_cu;
  if (max_tiles < grid) grid = max_tiles < 1 ? 1 : max_tiles;
  hipLaunchKernelGGL((mx_gemm_kernel<MODE, WN, kCont>), dim3(grid), dim3(T::kThreads), 0, stream, a);
  AFD_CHECK_LAUNCH();
  return AFD_OK;
}

template <int MODE>
static int launch_mx_any(const MxGemmArgs& p, int max_row_tiles, hipStream_t stream) {
  if constexpr (MODE != kDown) {
    // the continuous ring (static walk) decodes the next tile two stages before the end and
    // reads what was copied at the first stage: three stages at least
    if (p.K / kImgK >= 3 && p.walk_ctr == nullptr) {
      if (p.N % MxTile<4>::kBN == 0) return launch_mx<MODE, 4, true>(p, max_row_tiles, stream);
      return launch_mx<MODE, 2, true>(p, max_row_tiles, stream);
    }
  }
  if (p.N % MxTile<4>::kBN == 0) return launch_mx<MODE, 4, false>(p, max_row_tiles, stream);
  return launch_mx<MODE, 2, false>(p, max_row_tiles, stream);
}

int launch_mx_gate_up(const afd_moe_cfg& cfg, const afd_expert_weights& wt, uint8_t* ws,
                      const afd_ws_layout& L, const uint8_t* xq, const void* xs,
                      const afd_job* rows_desc, hipStream_t stream) {
  MxGemmArgs p;
  p.a_img = nullptr;
  p.a_rows = xq;
  p.a_scales = static_cast<const uint8_t*>(xs);
  p.rows_desc = rows_desc;
  p.topk = cfg.topk;
  p.topk_magic = div_magic(cfg.topk);
  p.act = act_params(cfg);
  p.b_img = static_cast<const uint8_t*>(wt.w13);
  p.sorted_pairs = reinterpret_cast<const int32_t*>(ws + L.sorted_pairs);
  p.tile_expert = reinterpret_cast<const int32_t*>(ws + L.tile_expert);
  p.num_tiles = reinterpret_cast<const int32_t*>(ws + L.num_tiles);
  p.padded_offsets = reinterpret_cast<const int32_t*>(ws + L.padded_offsets);
  p.counts = reinterpret_cast<const int32_t*>(ws + L.counts);
  p.walk_ctr = cfg.tile_walk == AFD_WALK_DYNAMIC ? call_counters(ws, L) + kGateUpWalkWord : nullptr;
  p.K = cfg.hidden;
  p.N = 2 * cfg.inter;
  p.h_img = ws + L.hq;
  p.y = nullptr;
  return cfg.activation != AFD_ACT_SWIGLU ? launch_mx_any<kGateUpParam>(p, L.max_tiles, stream)
                                         : launch_mx_any<kGateUp>(p, L.max_tiles, stream);
}

int launch_mx_down(const afd_moe_cfg& cfg, const afd_expert_weights& wt, uint8_t* ws,
                   const afd_ws_layout& L, int32_t n, hipStream_t stream) {
  (void)n;
  MxGemmArgs p;
  p.act = act_params(cfg);
  p.a_img = ws + L.hq;
  p.a_rows = nullptr;
  p.a_scales = nullptr;
  p.rows_desc = nullptr;
  p.topk = cfg.topk;
  p.topk_magic = div_magic(cfg.topk);
  p.b_img = static_cast<const uint8_t*>(wt.w2);
  p.sorted_pairs = reinterpret_cast<const int32_t*>(ws + L.sorted_pairs);
  p.tile_expert = reinterpret_cast<const int32_t*>(ws + L.tile_expert);
  p.num_tiles = reinterpret_cast<const int32_t*>(ws + L.num_tiles);
  p.padded_offsets = reinterpret_cast<const int32_t*>(ws + L.padded_offsets);
  p.counts = reinterpret_cast<const int32_t*>(ws + L.counts);
  p.walk_ctr = cfg.tile_walk == AFD_WALK_DYNAMIC ? call_counters(ws, L) + kDownWalkWord : nullptr;
  p.K = cfg.inter;
  p.N = cfg.hidden;
  p.h_img = nullptr;
  p.y = reinterpret_cast<uint16_t*>(ws + L.y);
  return launch_mx_any<kDown>(p, L.max_tiles, stream);
}

}  // namespace afd
