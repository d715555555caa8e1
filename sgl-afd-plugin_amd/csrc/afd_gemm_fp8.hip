// Grouped FP8-e4m3 GEMMs with 128x128-block fp32 weight scales and 1x128 fp32 activation
// scales (the block-FP8 expert format) on gfx950 MFMA (v_mfma_scale_f32_32x32x64_f8f6f4 with
// unit scales, e4m3 x e4m3).
//
//   gate_up: h[p, :] = silu(x_t . Wg_e^T) * (x_t . Wu_e^T) for every padded row p of expert e
//            (t = token of the pair at row p), quantized to e4m3 with one fp32 scale per 1x128
//            group (the down GEMM's A operand and its scales).
//   down:    y[p, :] = bf16(h_p . W2_e^T).
//
// Block scales: a 128-wide K stage kb is exactly one scale block of both operands, with the
// product s_kb = s_x[row, kb] * s_w[block, kb]; the result is sum_kb s_kb * P_kb, P_kb the
// stage's unscaled MFMA sum. The accumulators hold R_kb = (sum_{k <= kb} s_k P_k) / s_kb: before
// stage kb's MFMAs they are multiplied by s_{kb-1} / s_kb, the MFMAs then add P_kb, and the
// epilogue multiplies by the last s. This costs no second set of registers for the partial
// sums and one multiply per accumulator and stage; it rounds differently from folding each
// stage separately by about one fp32 rounding per stage (relative 2^-24 each). The MFMA
// operands are swapped (weights first, activations second), so a lane's accumulators all
// belong to one activation row and s_kb is one value per 32x32 tile.
//
// Tiling: a workgroup of 8 wavefronts owns a 128 x 256 output tile; wavefront (g, c) owns rows
// [64 g, 64 g + 64) and columns [64 c, 64 c + 64): 2 x 2 MFMA tiles, 64 accumulators per lane. Both operands move HBM -> LDS with gfx950's direct global_load_lds in
// 1 KiB pieces of 8 rows x 128 B, each lane fetching one 16-byte chunk of a row at its own
// offset, so the activation rows are gathered (gate_up: the token rows through sorted_pairs;
// down: the tile's rows of h) and the weight rows come straight from the [E][N][K] layout. LDS
// holds every operand in the swizzled 128-byte-row layout of the MX kernel's A images (no bank
// conflicts for the MFMA operand reads), in a ring of 3 stages. As in the MX kernel, the two
// wavefronts of a SIMD (group 0: rows 0-63, group 1: rows 64-127) ping-pong between reading a
// stage from LDS and running its 8 MFMAs (and rescaling its accumulators), half a stage
// apart. The persistent workgroups walk the tiles XCD by XCD in blocks of 8 x 4 tiles
// (TileWalk).
#include <type_traits>

#include "afd_common.h"
#include "afd_internal.h"

namespace afd {
namespace fp8 {

// gate_up with SwiGLU, gate_up with an activation that takes constants (SiTU, or SwiGLU with
// a limit: SiTU's longer epilogue would raise the register pressure of the SwiGLU kernel),
// down
enum { kGateUp = 0, kDown = 1, kGateUpParam = 2 };

// Tile walk blocks of 8 row tiles x 4 column tiles: a 1 MiB weight slice is shared 8 ways
// (column-tile-fastest walks fetch ~3x more from beyond L2).
constexpr int kWalkRows = 8;

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kBM = kBlockM;  // 128 activation rows
constexpr int kBN = 256;      // weight rows (output columns)
constexpr int kBK = 128;      // K per stage = one scale block
// LDS stage: activations (128 rows x 128 B), their 128 fp32 scales, weights (256 rows x 128 B)
constexpr int kXScales = kBM * kBK;         // 16384
constexpr int kWOff = kXScales + kBM * 4;   // 16896
constexpr int kStage = kWOff + kBN * kBK;   // 49664
constexpr int kStages = 3;
// after the ring: the tile's weight block scales for every K stage, two blocks x 32 stages
// per 256 B group (written by one wavefront's dword copies)
constexpr int kWScales = kStages * kStage;
constexpr int kMaxKT = 128;
// then the gate_up epilogue's per-row amax of each column wavefront, [128 rows][4]
constexpr int kAmax = kWScales + 2 * kMaxKT * 4;
constexpr int kLds = kAmax + kBM * 4 * 4;
// copies per wavefront and stage: 2 activation pieces, 4 weight pieces and one piece of
// activation scales (a wavefront past the two halves repeats its first weight piece: the same
// bytes to the same place), so every wavefront counts the same number of copies
constexpr int kQX = kBM / 8 / kWaves;  // 2
constexpr int kQW = kBN / 8 / kWaves;  // 4
constexpr int kPieces = kQX + kQW + 1;
// the down epilogue's bf16 tile: kBM rows of kBN / 8 16-byte chunks, chunk c of row r at
// physical chunk c ^ (r % 16), so the 16 rows a 16-lane pass of a write covers (one logical
// chunk each) and the 16 consecutive chunks a pass of a read covers (one row) fall on 16
// distinct 16-byte bank groups
constexpr int kYChunks = kBN / 8;
static_assert(kQX * kWaves * 8 == kBM && kQW * kWaves * 8 == kBN, "pieces cover the tile");
static_assert(kBM * kBN * 2 <= kStages * kStage, "down epilogue tile must fit the stages");
static_assert(kLds <= 160 * 1024, "LDS of one CU");
static_assert(2 * kPieces < 64, "vmcnt is a 6-bit counter");

struct Fp8GemmArgs {
  const uint8_t* a;   // gate_up: token rows xq [n][K]; down: hq [np][K]
  const float* as;    // their scales: xs [n][K/128]; hs [np][K/128]
  const afd_job* rows_desc;  // gate_up: if set, a / as are its xq / xs
  int topk;
  uint32_t topk_magic;  // div_magic(topk)
  const uint8_t* b;     // e4m3 [E][N][K] (gate_up rows interleaved gate/up by 32)
  const float* bs;      // [E][N/128][K/128] in logical block order
  const int32_t* sorted_pairs;    // [np] flat pair index per padded row, -1 = pad
  const int32_t* tile_expert;     // [row tiles]
  const int32_t* num_tiles;       // [1]
  const int32_t* padded_offsets;  // [E + 1]
  const int32_t* counts;          // [E]
  uint32_t* walk_ctr;             // [8] zeroed tile counters (one per XCD); nullptr: static walk
  int K, N;
  ActParams act;  // gate_up: the activation
  uint8_t* hq;  // gate_up out: e4m3 [np][N/2]
  float* hs;    // gate_up out: fp32 [np][N/256]
  uint16_t* y;  // down out: bf16 [np][N]
};

template <int MODE>
__global__ __launch_bounds__(kThreads) void fp8_gemm_kernel(Fp8GemmArgs p) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kLds];
  const int t = threadIdx.x, lane = t & 63;
  const int w_u = __builtin_amdgcn_readfirstlane(t >> 6);  // wavefront index, scalar
  const int wm = w_u / 4, wn = w_u % 4, lr = lane & 31, lk = lane >> 5;
  const TileWalk<kWalkRows> walk(p.num_tiles[0], p.N / kBN, blockIdx.x, gridDim.x, p.walk_ctr);
  __shared__ int claimed[2];  // the claimed walk positions lane 0 publishes (as in the MX kernel)
  const int KT = p.K / kBK;
  const int nblk = p.N / kBK;  // weight scale blocks along N
  const uint32_t lds_base = __builtin_amdgcn_readfirstlane(lds_offset(lds));

  // Copy offsets. Piece q of a wavefront covers 8 rows: image row r = 8 (w Q + q) + lane / 8,
  // physical chunk lane % 8, i.e. logical chunk (lane % 8) ^ swizzle(r) of the source row.
  // Weight rows and down's h rows are fixed per lane (the tile is a scalar base); gate_up's
  // rows are token rows, looked up per tile. Wavefronts 0 and 1 also copy the activation
  // scales of rows [64 w, 64 w + 64).
  auto chunk = [&](int r) { return (lane & 7) ^ ((r ^ (r >> 3)) & 7); };
  uint32_t w_voff[kQW];
#pragma unroll
  for (int q = 0; q < kQW; ++q) {
    const int r = 8 * (w_u * kQW + q) + (lane >> 3);
    w_voff[q] = static_cast<uint32_t>(r * p.K + chunk(r) * 16);
  }
  const bool copies_scales = w_u < 2;
  const int s_row = 64 * (w_u & 1) + lane;

  // A tile's metadata is loaded one tile ahead and decoded after the previous tile's K loop,
  // whose last wait leaves no copy in flight, so no tile starts by waiting for a load.
  int sp_next[kQX + 1], e_next = 0;
  auto load_next = [&](int ii) {
    int m, nn;
    walk.at_dense(ii, m, nn);
    e_next = p.tile_expert[m];
    if constexpr (MODE != kDown) {
#pragma unroll
      for (int q = 0; q < kQX; ++q)
        sp_next[q] = p.sorted_pairs[m * kBM + 8 * (w_u * kQX + q) + (lane >> 3)];
      sp_next[kQX] = p.sorted_pairs[m * kBM + s_row];
    }
  };
  int e_cur = 0;
  uint32_t x_voff[kQX], s_voff;
  // down: rows of the tile, relative to the tile's first row
#pragma unroll
  for (int q = 0; q < kQX; ++q) {
    const int r = 8 * (w_u * kQX + q) + (lane >> 3);
    x_voff[q] = static_cast<uint32_t>(r * p.K + chunk(r) * 16);
  }
  s_voff = static_cast<uint32_t>(s_row * KT * 4);
  auto decode_next = [&]() {
    e_cur = __builtin_amdgcn_readfirstlane(e_next);
    if constexpr (MODE != kDown) {
      // padding rows (-1) read token 0; their results are never used
      auto token = [&](int sp) {
        return sp >= 0 ? div_by_magic(static_cast<uint32_t>(sp), p.topk_magic) : 0u;
      };
#pragma unroll
      for (int q = 0; q < kQX; ++q) {
        const int r = 8 * (w_u * kQX + q) + (lane >> 3);
        x_voff[q] = token(sp_next[q]) * static_cast<uint32_t>(p.K) + chunk(r) * 16;
      }
      s_voff = token(sp_next[kQX]) * static_cast<uint32_t>(KT * 4);
    }
  };
  // The tile whose stages the copies below fetch. gate_up starts the next tile's copies
  // (weight scales and the first two stages) right after its own K loop: its epilogue works
  // from registers and a small LDS area outside the ring, so the copies land while it runs.
  // down's epilogue stages its output through the ring, so it starts them at the tile start.
  constexpr bool kEarlyStart = MODE != kDown;
  const uint8_t* x_tile = nullptr;
  const float* s_tile = nullptr;
  const uint8_t* w_tile = nullptr;
  int blk0 = 0, blk1 = 0;
  int64_t e_copy = 0;
  const uint8_t* a_rows = p.a;
  const float* a_scales = p.as;
  if (MODE != kDown && p.rows_desc != nullptr) {
    a_rows = p.rows_desc->xq;
    a_scales = static_cast<const float*>(p.rows_desc->xs);
  }
  auto copy_tile = [&](int mt, int nt, int64_t e) {
    x_tile = MODE != kDown ? a_rows : a_rows + int64_t(mt) * kBM * p.K;
    s_tile = MODE != kDown ? a_scales : a_scales + int64_t(mt) * kBM * KT;
    w_tile = p.b + (e * p.N + int64_t(nt) * kBN) * int64_t(p.K);
    // the two weight scale blocks of the tile: gate_up (gate, up) of its 128 h columns;
    // down the two 128-row blocks (wavefront columns 64 c use block c / 2)
    blk0 = MODE != kDown ? nt * kBN / 256 : nt * kBN / 128;
    blk1 = MODE != kDown ? nblk / 2 + nt * kBN / 256 : nt * kBN / 128 + 1;
    e_copy = e;
  };
  auto issue_piece = [&](int kt, auto qc) {
    constexpr int q = decltype(qc)::value;
    const uint32_t st = lds_base + static_cast<uint32_t>((kt % kStages) * kStage);
    if constexpr (q < kQX) {
      lds_dma16(st + (w_u * kQX + q) * 1024, x_tile + kt * kBK, x_voff[q]);
    } else if constexpr (q < kQX + kQW) {
      constexpr int qw = q - kQX;
      lds_dma16(st + kWOff + (w_u * kQW + qw) * 1024, w_tile + kt * kBK, w_voff[qw]);
    } else {
      if (copies_scales)
        lds_dma4(st + kXScales + (w_u & 1) * 256, s_tile + kt, s_voff);
      else
        lds_dma16(st + kWOff + w_u * kQW * 1024, w_tile + kt * kBK, w_voff[0]);
    }
  };
  auto issue = [&](int kt) { static_for<kPieces>([&](auto q) { issue_piece(kt, q); }); };
  const int last = KT - 1;
  // Wavefront 0 first copies the tile's weight block scales (lane x: block x < 32 ? blk0 :
  // blk1, stage 32 g + x % 32, clamped in bounds); those copies are older than every piece of
  // stage 0, so the wait for stage 0 covers them. Then the first two stages.
  auto start_copies = [&]() {
    if (w_u == 0) {
      const float* bs_e = p.bs + e_copy * nblk * KT;
      const int b = lk == 0 ? blk0 : blk1;
      for (int g = 0; g * 32 < KT; ++g) {
        const int kb = min(lr + 32 * g, KT - 1);
        lds_dma4(lds_base + kWScales + g * 256, bs_e, static_cast<uint32_t>((b * KT + kb) * 4));
      }
    }
    issue(0);
    issue(min(1, last));
  };

  // The walk's dense positions: static, or with p.walk_ctr claimed one tile ahead by lane 0
  // (the first two here, each later one during the last K stage of the tile before the one
  // that needs it); see the MX kernel.
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
  if (i < walk.tiles) {
    load_next(i);
    decode_next();
    if constexpr (kEarlyStart) {
      int mt, nt;
      walk.at_dense(i, mt, nt);
      copy_tile(mt, nt, e_cur);
      start_copies();
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
    if (has_next) load_next(i_next);
    if constexpr (!kEarlyStart) copy_tile(mt, nt, e);

    v16f acc[2][2];
#pragma unroll
    for (int i2 = 0; i2 < 2; ++i2)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 16; ++q) acc[i2][j][q] = 0.0f;

    // Operand fragments of both k-steps of one stage and the stage's scales. An 8-bit operand
    // lane half h holds K [16h, 16h+16) in bytes 0-15 and K [32+16h, 32+16h+16) in bytes 16-31
    // of the k-step. x: activation rows 64 g + 32 i + lane % 32; w: weight rows
    // 64 c + 32 j + lane % 32.
    struct Frag {
      v8i x[2][2], w[2][2];  // [ks][i], [ks][j]
      float sx[2], sw[2];
    };
    Frag f;
    float sx_prev[2] = {1.0f, 1.0f}, sw_prev[2] = {1.0f, 1.0f};
    const float* wsc = reinterpret_cast<const float*>(lds + kWScales);
    auto read_stage = [&](int kt) {
      const uint8_t* xb = lds + (kt % kStages) * kStage;
      const uint8_t* wb = xb + kWOff;
      // row r + 32 has the swizzle of row r with chunk bit 2 flipped: its chunk c sits 4096 B
      // after row r's chunk c ^ 4, so four lane addresses serve both row blocks
      const int rx = wm * 64 + lr, rw = wn * 64 + lr;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
        for (int i2 = 0; i2 < 2; ++i2) {
          const int kc = (ks ^ i2) * 4 + lk;
          v4i lo = *reinterpret_cast<const v4i*>(xb + img_a_off(rx, kc) + i2 * 4096);
          v4i hi = *reinterpret_cast<const v4i*>(xb + img_a_off(rx, kc + 2) + i2 * 4096);
          f.x[ks][i2] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          lo = *reinterpret_cast<const v4i*>(wb + img_a_off(rw, kc) + i2 * 4096);
          hi = *reinterpret_cast<const v4i*>(wb + img_a_off(rw, kc + 2) + i2 * 4096);
          f.w[ks][i2] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
      }
      const float* sx = reinterpret_cast<const float*>(xb + kXScales);
      f.sx[0] = sx[wm * 64 + lr];
      f.sx[1] = sx[wm * 64 + 32 + lr];
      // block b of stage kt at group kt / 32, half b, word kt % 32
      const float* sw = wsc + (kt >> 5) * 64 + (kt & 31);
      if constexpr (MODE != kDown) {
        f.sw[0] = sw[0];
        f.sw[1] = sw[32];
      } else {
        f.sw[0] = f.sw[1] = sw[(wn >> 1) * 32];
      }
    };
    // The stage's 8 MFMAs. Before its first k-step, a tile's accumulators go from R_{kb-1} to
    // R_{kb-1} * s_{kb-1} / s_kb (stage kb's scales are in f); those 16 multiplies overlap the
    // previous tiles' MFMAs. On the first stage the accumulators are 0 and the ratio is unused.
    auto mma_stage = [&]() {
      float ratio[2][2];
#pragma unroll
      for (int i2 = 0; i2 < 2; ++i2)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          ratio[i2][j] = (sx_prev[i2] * sw_prev[j]) * __builtin_amdgcn_rcpf(f.sx[i2] * f.sw[j]);
      static_for<2>([&](auto ksc) {
        constexpr int ks = decltype(ksc)::value;
        static_for<2>([&](auto i2c) {
          constexpr int i2 = decltype(i2c)::value;
          static_for<2>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            if constexpr (ks == 0) {
#pragma unroll
              for (int q = 0; q < 16; ++q) acc[i2][j][q] *= ratio[i2][j];
            }
            // D[weight row][activation row]: lane x holds activation row x % 32
            acc[i2][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                f.w[ks][j], f.x[ks][i2], acc[i2][j], 0 /*e4m3*/, 0 /*e4m3*/, 0, 127 /*x1*/, 0,
                127 /*x1*/);
          });
        });
      });
      sx_prev[0] = f.sx[0];
      sx_prev[1] = f.sx[1];
      sw_prev[0] = f.sw[0];
      sw_prev[1] = f.sw[1];
    };

    // Ping-pong as in the MX kernel: each group copies its pieces of stage kt+2 when it starts
    // reading stage kt; copies are clamped to the last stage (a clamped copy rewrites a slot
    // with its own bytes). Epilogue stores of the previous tile still in flight only make the
    // counted waits stricter (loads complete in order among themselves).
    if constexpr (!kEarlyStart) start_copies();
    wait_vmcnt<kPieces>();  // own pieces of stage 0 (and the weight scales) landed
    __syncthreads();
    if (wm == 0) {
      for (int kt = 0; kt < KT; ++kt) {
        // the claim rides on the last stage, whose end waits for every copy anyway
        if (claims && kt == last) ticket = walk.claim_ticket();
        issue(min(kt + 2, last));
        read_stage(kt);
        wait_vmcnt_lds<2 * kPieces>();  // own reads done (copies may be in flight)
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(1);
        mma_stage();
        __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt<kPieces>();  // own pieces of stage kt+1 landed
        __syncthreads();
      }
      __syncthreads();
    } else {
      __syncthreads();
      for (int kt = 0; kt < KT; ++kt) {
        issue(min(kt + 2, last));
        read_stage(kt);
        wait_vmcnt_lds<kPieces>();  // own reads done, own pieces of stage kt+1 landed
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(1);
        mma_stage();
        __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
      }
    }
    // R_last * s_last
#pragma unroll
    for (int i2 = 0; i2 < 2; ++i2)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float sl = sx_prev[i2] * sw_prev[j];
#pragma unroll
        for (int q = 0; q < 16; ++q) acc[i2][j][q] *= sl;
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
        start_copies();
      }
    }

    // accumulator q of tile (i, j): activation row 64 g + 32 i + lane % 32, output column
    // 64 c + 32 j + 8 (q / 4) + 4 (lane / 32) + q % 4
    if constexpr (MODE != kDown) {
      // SwiGLU (or SiTU) in registers: column tiles j = 0, 1 are the gate and up halves of one
      // 64-row group of interleaved W13, i.e. the same 32 intermediate columns; the lane holds
      // h columns 32 c + 8 q4 + 4 lk + (0..3) of its two rows. The tile's 128 h columns are
      // one 1x128 group per row: the row's amax over its 4 column wavefronts goes through a
      // 2 KiB LDS area; then each lane half assembles 16 contiguous codes with one exchange
      // and stores them.
      const int inter = p.N / 2;
      float* amax_l = reinterpret_cast<float*>(lds + kAmax);
      auto quant_store = [&](auto fn) {
        float h[2][16];
#pragma unroll
        for (int i2 = 0; i2 < 2; ++i2) {
          float m = 0.0f;
#pragma unroll
          for (int q = 0; q < 16; ++q) {
            h[i2][q] = fn(acc[i2][0][q], acc[i2][1][q]);
            m = fmaxf(m, fabsf(h[i2][q]));
          }
          m = fmaxf(m, xor32(m, lk));
          if (lk == 0) amax_l[(wm * 64 + i2 * 32 + lr) * 4 + wn] = m;
        }
        __syncthreads();
#pragma unroll
        for (int i2 = 0; i2 < 2; ++i2) {
          const int row = wm * 64 + i2 * 32 + lr;
          const v4f a4 = *reinterpret_cast<const v4f*>(amax_l + row * 4);
          const float amax = fmaxf(fmaxf(a4[0], a4[1]), fmaxf(a4[2], a4[3]));
          const float sc = fmaxf(amax, kFp8Eps) / kE4m3Max;
          uint32_t d[4];
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4)
            d[q4] = pk4_e4m3(h[i2][4 * q4] / sc, h[i2][4 * q4 + 1] / sc, h[i2][4 * q4 + 2] / sc,
                             h[i2][4 * q4 + 3] / sc);
          // lane half 0 takes columns 0-15 (its d0, d1 and the partner's), half 1 columns
          // 16-31 (the partner's d2, d3 and its own)
          const uint32_t p0 = swap_halves(d[2], d[0], lk);
          const uint32_t p1 = swap_halves(d[3], d[1], lk);
          v4i chunk;
          chunk[0] = static_cast<int>(lk ? p0 : d[0]);
          chunk[1] = static_cast<int>(lk ? d[2] : p0);
          chunk[2] = static_cast<int>(lk ? p1 : d[1]);
          chunk[3] = static_cast<int>(lk ? d[3] : p1);
          *reinterpret_cast<v4i*>(p.hq + int64_t(m0 + row) * inter + n0 / 2 + wn * 32 + lk * 16) =
              chunk;
          if (wn == 0 && lk == 0) p.hs[int64_t(m0 + row) * (inter / kBK) + n0 / 256] = sc;
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
    } else {
      // Lane half lk holds columns 8 q4 + 4 lk .. + 3 of each 32-column tile; trading halves
      // with v_permlane32_swap (first operand of lanes 32-63 for the second of lanes 0-31)
      // leaves lane half lk with whole 16-byte chunks 2 pr + lk, in column order, written to
      // LDS with one 16-byte write each.
      const int nvalid = min(kBM, row_end - m0);  // rows [0, nvalid) of this tile are real
      auto y_chunk = [](int r, int c) { return (r * kYChunks + (c ^ (r & 15))) * 16; };
#pragma unroll
      for (int i2 = 0; i2 < 2; ++i2)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int row = wm * 64 + i2 * 32 + lr;
          const v16f& a = acc[i2][j];
          uint32_t h[4][2];
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) {
            h[q4][0] = pk_bf16(a[q4 * 4], a[q4 * 4 + 1]);
            h[q4][1] = pk_bf16(a[q4 * 4 + 2], a[q4 * 4 + 3]);
          }
#pragma unroll
          for (int pr = 0; pr < 2; ++pr) {
            const auto d0 = __builtin_amdgcn_permlane32_swap(h[2 * pr][0], h[2 * pr + 1][0], false, false);
            const auto d1 = __builtin_amdgcn_permlane32_swap(h[2 * pr][1], h[2 * pr + 1][1], false, false);
            const v4i chunk = {static_cast<int>(d0[0]), static_cast<int>(d1[0]), static_cast<int>(d0[1]),
                               static_cast<int>(d1[1])};
            *reinterpret_cast<v4i*>(lds + y_chunk(row, (wn * 64 + j * 32) / 8 + 2 * pr + lk)) = chunk;
          }
        }
      __syncthreads();
#pragma unroll 4
      for (int q = 0; q < kBM * kYChunks / kThreads; ++q) {
        const int idx = q * kThreads + t;
        const int row = idx / kYChunks, c = idx % kYChunks;
        if (row < nvalid)
          __builtin_nontemporal_store(*reinterpret_cast<const v4i*>(lds + y_chunk(row, c)),
                                      reinterpret_cast<v4i*>(p.y + int64_t(m0 + row) * p.N + n0 + c * 8));
      }
      __syncthreads();
    }
  }
}

template <int MODE>
static int launch(Fp8GemmArgs p, int max_row_tiles, hipStream_t stream) {
  if (p.K % kBK || p.N % kBN || p.K / kBK > kMaxKT) return AFD_ERR_SHAPE;
  // resident workgroups per CU (registers and LDS decide); initialized once, thread-safely
  static const int per_cu = [] {
    int b = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, fp8_gemm_kernel<MODE>, kThreads, 0) !=
            hipSuccess ||
        b < 1)
      b = 1;
    return b;
  }();
  const int max_tiles = max_row_tiles * (p.N / kBN);
  int grid = device_cu_count() * per_cu;
  if (max_tiles < grid) grid = max_tiles < 1 ? 1 : max_tiles;
  hipLaunchKernelGGL(fp8_gemm_kernel<MODE>, dim3(grid), dim3(kThreads), 0, stream, p);
  AFD_CHECK_LAUNCH();
  return AFD_OK;
}

static Fp8GemmArgs common_args(const afd_moe_cfg& cfg, uint8_t* ws, const afd_ws_layout& L) {
  Fp8GemmArgs p;
  p.topk = cfg.topk;
  p.topk_magic = div_magic(cfg.topk);
  p.act = act_params(cfg);
  p.sorted_pairs = reinterpret_cast<const int32_t*>(ws + L.sorted_pairs);
  p.tile_expert = reinterpret_cast<const int32_t*>(ws + L.tile_expert);
  p.num_tiles = reinterpret_cast<const int32_t*>(ws + L.num_tiles);
  p.padded_offsets = reinterpret_cast<const int32_t*>(ws + L.padded_offsets);
  p.counts = reinterpret_cast<const int32_t*>(ws + L.counts);
  p.hq = nullptr;
  p.hs = nullptr;
  p.y = nullptr;
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
  p.rows_desc = nullptr;
  p.b = static_cast<const uint8_t*>(wt.w2);
  p.bs = static_cast<const float*>(wt.s2);
  p.walk_ctr = cfg.tile_walk == AFD_WALK_DYNAMIC ? call_counters(ws, L) + kDownWalkWord : nullptr;
  p.K = cfg.inter;
  p.N = cfg.hidden;
  p.y = reinterpret_cast<uint16_t*>(ws + L.y);
  return fp8::launch<fp8::kDown>(p, L.max_tiles, stream);
}

}  // namespace afd
