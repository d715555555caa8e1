// Routing of one job's (token, k) pairs to this F rank's local experts, on gfx950.
//
// Two launches, integer work on a 4*n*k-byte id array (HBM/latency bound):
//   1. route_prep:    workgroup c < chunks histograms chunk c of the flat pair array by local
//                     expert (LDS atomics; counts are order-free); with the expert call, the
//                     remaining workgroups quantize the activations meanwhile (afd_quant_dev.h).
//   2. route_scatter: workgroup c first reads the whole histogram (it is in L2; stored expert
//                     by expert, [E][kMaxChunks], so each thread's run of chunk counts is a few
//                     16-byte loads issued together) to get each expert's count, its own chunk's
//                     base per expert and the block_m-padded expert offsets (a wavefront scan);
//                     workgroup 0 also writes
//                     counts, offsets, padded offsets, the row-tile table, the tile count and
//                     the -1 fill of padding rows. It then walks its pairs in flat order, 256 at
//                     a time; a pair's rank among equal keys inside its wavefront comes from 9
//                     ballots (one per key bit), across wavefronts from LDS counts, so the
//                     placement is the stable order (ascending flat index inside each expert)
//                     bit for bit.
#include "afd_common.h"
#include "afd_internal.h"
#include "afd_quant_dev.h"

namespace afd {

constexpr int kRouteThreads = 256;
constexpr int kMaxChunks = 128;
constexpr int kKeyBits = 9;  // keys 0..256 (local expert, or num_local for "not local")
static_assert(kRouteThreads == kQuantThreads, "the prep kernel's workgroups do either job");

__device__ __forceinline__ int pair_key(int id, int e_lo, int num_local) {
  unsigned rel = static_cast<unsigned>(id - e_lo);
  return rel < static_cast<unsigned>(num_local) ? static_cast<int>(rel) : num_local;
}

// activation quantization run by the prep kernel beside the histogram
enum { kPrepNone = 0, kPrepMxfp8 = 1, kPrepFp8 = 2 };
struct PrepQuant {
  int cols;  // items: n * cols / 32 MX blocks (MXFP8) or quarter groups (FP8 1x128)
  uint8_t* q;
  void* s;
};

template <int QUANT>
__global__ __launch_bounds__(kRouteThreads) void route_prep_kernel(
    JobIn jin, int topk, int chunk, int chunks, int e_lo, int num_local,
    int32_t* __restrict__ hist, PrepQuant pq, uint32_t* __restrict__ counters) {
  const JobIn job = resolve_job(jin);
  if (blockIdx.x == 0 && threadIdx.x < kCounterLines) {
    uint32_t* line = counters + kLineWord0 + threadIdx.x * kLineStride;
    line[0] = line[1] = line[2] = 0u;
    if (threadIdx.x == 0) counters[kArriveWord] = 0u;
  }
  if (static_cast<int>(blockIdx.x) >= chunks) {
    const int64_t first = (int64_t(blockIdx.x) - chunks) * kRouteThreads + threadIdx.x;
    const int64_t stride = (int64_t(gridDim.x) - chunks) * kRouteThreads;
    const int64_t items = job.n * (pq.cols / kMxBlock);
    const int cols = pq.cols;
    auto xrow = [&job, cols](int64_t r) { return job_x_row(job, r, cols); };
    if constexpr (QUANT == kPrepMxfp8)
      quant_mxfp8_items<true>(xrow, items, cols, pq.q, static_cast<uint8_t*>(pq.s), first, stride);
    else if constexpr (QUANT == kPrepFp8)
      quant_fp8_1x128_items(xrow, items, cols, pq.q, static_cast<float*>(pq.s), first, stride);
    return;
  }
  const int64_t pairs = job.n * topk;
  __shared__ int cnt[kMaxLocalExperts];
  for (int e = threadIdx.x; e < num_local; e += kRouteThreads) cnt[e] = 0;
  __syncthreads();
  const int64_t lo = int64_t(blockIdx.x) * chunk;
  const int64_t hi = lo + chunk < pairs ? lo + chunk : pairs;
  for (int64_t i = lo + threadIdx.x; i < hi; i += kRouteThreads) {
    int key = pair_key(job_id(job, i, topk), e_lo, num_local);
    if (key < num_local) atomicAdd(&cnt[key], 1);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < num_local; e += kRouteThreads)
    hist[int64_t(e) * kMaxChunks + blockIdx.x] = cnt[e];
}

__global__ __launch_bounds__(kRouteThreads) void route_scatter_kernel(
    JobIn jin, int topk, int chunk, int chunks, int e_lo, int num_local, int block_m,
    const int32_t* __restrict__ hist, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ poff, int32_t* __restrict__ sorted_pairs,
    int32_t* __restrict__ pair_pos, int32_t* __restrict__ tile_expert,
    int32_t* __restrict__ num_tiles) {
  const JobIn job = resolve_job(jin);
  const int64_t pairs = job.n * topk;
  constexpr int kWaves = kRouteThreads / 64;
  __shared__ int run[kMaxLocalExperts + 1];
  __shared__ int wcnt[kWaves][kMaxLocalExperts + 1];
  __shared__ int part_all[kRouteThreads], part_before[kRouteThreads];
  __shared__ int tot[kMaxLocalExperts];
  __shared__ int pof[kMaxLocalExperts + 1];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int c = blockIdx.x;
  const int64_t lo = int64_t(c) * chunk;
  const int64_t hi = lo + chunk < pairs ? lo + chunk : pairs;
  // the chunk's first two batches of 256 ids are loaded now, so their latency overlaps the
  // histogram pass; each later batch is loaded two batches ahead
  int id_cur = lo + t < hi ? job_id(job, lo + t, topk) : 0;
  int id_nxt = lo + kRouteThreads + t < hi ? job_id(job, lo + kRouteThreads + t, topk) : 0;
  // Expert e's chunks are split over G = kRouteThreads / num_local threads (e, g), each summing
  // a contiguous run of them (a multiple of 4 long, so 16-byte loads of the expert's row of the
  // histogram; entries at or past `chunks` are never written and are masked): the counts in
  // all chunks and in the chunks before this one.
  const int G = kRouteThreads / num_local;
  const int per = ((chunks + G - 1) / G + 3) & ~3;
  const int e = t % num_local, g = t / num_local;
  const bool active = g < G;
  const int c0 = active ? g * per : 0, c1 = active ? min(c0 + per, chunks) : 0;
  int all = 0, before = 0;
  const int32_t* hrow = hist + int64_t(e) * kMaxChunks;
#pragma unroll 8
  for (int k4 = c0; k4 < c1; k4 += 4) {
    const v4i h = *reinterpret_cast<const v4i*>(hrow + k4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int v = k4 + j < c1 ? h[j] : 0;
      all += v;
      before += k4 + j < c ? v : 0;
    }
  }
  part_all[t] = all;
  part_before[t] = before;
  for (int i = t; i < kWaves * (kMaxLocalExperts + 1); i += kRouteThreads) (&wcnt[0][0])[i] = 0;
  __syncthreads();
  if (active && g == 0) {
    int a = 0, b = 0;
    for (int h = 0; h < G; ++h) {
      a += part_all[h * num_local + e];
      b += part_before[h * num_local + e];
    }
    tot[e] = a;
    run[e] = b;  // this chunk's rank base inside expert e; the segment start is added below
  }
  __syncthreads();
  // expert offsets and block_m-padded offsets: one wavefront, 4 experts per lane
  if (t < 64) {
    int o[4], q[4], so = 0, sp = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ex = t * 4 + i;
      const int n_e = ex < num_local ? tot[ex] : 0;
      o[i] = so;
      q[i] = sp;
      so += n_e;
      sp += (n_e + block_m - 1) / block_m * block_m;
    }
    int io = so, ip = sp;  // inclusive scans of the lane totals
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int vo = __shfl_up(io, d), vp = __shfl_up(ip, d);
      if (t >= d) {
        io += vo;
        ip += vp;
      }
    }
    const int bo = io - so, bp = ip - sp;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ex = t * 4 + i;
      if (ex < num_local) {
        pof[ex] = bp + q[i];
        if (c == 0) {
          counts[ex] = tot[ex];
          offsets[ex] = bo + o[i];
          poff[ex] = bp + q[i];
        }
      }
    }
    if (t == 63) {
      pof[num_local] = ip;
      if (c == 0) {
        offsets[num_local] = io;
        poff[num_local] = ip;
        num_tiles[0] = ip / block_m;
      }
    }
  }
  __syncthreads();
  for (int ex = t; ex < num_local; ex += kRouteThreads) run[ex] += pof[ex];
  if (c == 0) {
    // row-tile table (thread e writes expert e's tiles) and -1 on the padding rows of every
    // segment (the G threads of expert e stride over its at most block_m - 1 padding rows)
    if (t < num_local)
      for (int i = pof[t] / block_m, i1 = pof[t + 1] / block_m; i < i1; ++i) tile_expert[i] = t;
    if (active)
      for (int r = pof[e] + tot[e] + g; r < pof[e + 1]; r += G) sorted_pairs[r] = -1;
  }
  __syncthreads();
  const uint64_t below = (uint64_t(1) << lane) - 1;
  for (int64_t base = lo; base < hi; base += kRouteThreads) {
    const int64_t i = base + t;
    const bool live = i < hi;
    const int id = id_cur;
    id_cur = id_nxt;
    id_nxt = i + 2 * kRouteThreads < hi ? job_id(job, i + 2 * kRouteThreads, topk) : 0;
    const int key = live ? pair_key(id, e_lo, num_local) : num_local;
    // lanes with the same key (dead lanes join the "not local" key and are ignored)
    uint64_t peers = __ballot(1);
#pragma unroll
    for (int b = 0; b < kKeyBits; ++b) {
      uint64_t m = __ballot((key >> b) & 1);
      peers &= ((key >> b) & 1) ? m : ~m;
    }
    const int rank = __popcll(peers & below);
    if (rank == 0 && key < num_local) wcnt[wave][key] = __popcll(peers);
    __syncthreads();
    if (live) {
      if (key < num_local) {
        int pos = run[key] + rank;
        for (int w = 0; w < wave; ++w) pos += wcnt[w][key];
        sorted_pairs[pos] = static_cast<int32_t>(i);
        pair_pos[i] = pos;
      } else {
        pair_pos[i] = -1;
      }
    }
    __syncthreads();
    for (int e = t; e < num_local; e += kRouteThreads) {
      int add = 0;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        add += wcnt[w][e];
        wcnt[w][e] = 0;
      }
      run[e] += add;
    }
    __syncthreads();
  }
}

// Chunking of the flat pair array: at most kMaxChunks chunks of a multiple of 256 pairs.
void route_chunking(int64_t pairs, int* chunks, int* chunk) {
  int64_t c = (pairs + kMaxChunks - 1) / kMaxChunks;
  c = (c + kRouteThreads - 1) / kRouteThreads * kRouteThreads;
  if (c < kRouteThreads) c = kRouteThreads;
  *chunk = static_cast<int>(c);
  *chunks = pairs == 0 ? 0 : static_cast<int>((pairs + c - 1) / c);
}

int launch_route_quant(const JobIn& job, bool quantize, const afd_moe_cfg& cfg, uint8_t* ws,
                       const afd_ws_layout& L, hipStream_t stream, hipEvent_t mid) {
  uint32_t* counters = call_counters(ws, L);
  // grids for job.n tokens (with a descriptor: n_cap; chunks past the job's pairs are empty)
  const int64_t pairs = job.n * cfg.topk;
  int chunks, chunk;
  route_chunking(pairs, &chunks, &chunk);
  int32_t* hist = reinterpret_cast<int32_t*>(ws + L.hist);
  PrepQuant pq{cfg.hidden, ws + L.xq, ws + L.xs};
  int quant_grid = 0;
  const int fmt = !quantize ? kPrepNone : cfg.weight_fmt == AFD_W_MXFP4 ? kPrepMxfp8 : kPrepFp8;
  if (fmt != kPrepNone) quant_grid = grid_for(job.n * (cfg.hidden / kMxBlock));
  if (job.n > 0 && chunks + quant_grid > 0) {
    const dim3 grid(chunks + quant_grid);
    if (fmt == kPrepMxfp8)
      hipLaunchKernelGGL(route_prep_kernel<kPrepMxfp8>, grid, dim3(kRouteThreads), 0, stream, job,
                         cfg.topk, chunk, chunks, cfg.expert_lo, cfg.num_local, hist, pq, counters);
    else if (fmt == kPrepFp8)
      hipLaunchKernelGGL(route_prep_kernel<kPrepFp8>, grid, dim3(kRouteThreads), 0, stream, job,
                         cfg.topk, chunk, chunks, cfg.expert_lo, cfg.num_local, hist, pq, counters);
    else
      hipLaunchKernelGGL(route_prep_kernel<kPrepNone>, grid, dim3(kRouteThreads), 0, stream, job,
                         cfg.topk, chunk, chunks, cfg.expert_lo, cfg.num_local, hist, pq, counters);
    AFD_CHECK_LAUNCH();
  }
  if (mid) AFD_CHECK_HIP(hipEventRecord(mid, stream));
  // at least one workgroup, which writes the (empty) tables when there are no pairs
  hipLaunchKernelGGL(route_scatter_kernel, dim3(chunks > 0 ? chunks : 1), dim3(kRouteThreads), 0,
                     stream, job, cfg.topk, chunk, chunks, cfg.expert_lo, cfg.num_local,
                     L.block_m, hist, reinterpret_cast<int32_t*>(ws + L.counts),
                     reinterpret_cast<int32_t*>(ws + L.offsets),
                     reinterpret_cast<int32_t*>(ws + L.padded_offsets),
                     reinterpret_cast<int32_t*>(ws + L.sorted_pairs),
                     reinterpret_cast<int32_t*>(ws + L.pair_pos),
                     reinterpret_cast<int32_t*>(ws + L.tile_expert),
                     reinterpret_cast<int32_t*>(ws + L.num_tiles));
  AFD_CHECK_LAUNCH();
  return AFD_OK;
}

}  // namespace afd

extern "C" int afd_route(const int32_t* ids, int32_t n, const afd_moe_cfg* cfg, void* ws,
                         uint64_t ws_bytes, afd_stream_t stream) {
  afd_ws_layout L;
  int st = afd_workspace_layout(cfg, n, &L);
  if (st != AFD_OK) return st;
  if ((!ids && n > 0) || !ws) return AFD_ERR_ARG;
  if (ws_bytes < L.total) return AFD_ERR_WORKSPACE;
  const afd::JobIn job{nullptr, nullptr, ids, nullptr, nullptr, n};
  return afd::launch_route_quant(job, false, *cfg, static_cast<uint8_t*>(ws), L,
                                 static_cast<hipStream_t>(stream), nullptr);
}
