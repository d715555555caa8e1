// Routing of one job's (token, k) pairs to this F rank's local experts, on gfx950.
//
// Three small launches, all integer work on a 4*n*k-byte id array (HBM/latency bound):
//   1. route_hist:    chunk c of the flat pair array -> per-chunk expert histogram (LDS
//                     atomics; counts are order-free).
//   2. route_scan:    one workgroup turns the [chunks][E] histogram into per-chunk exclusive
//                     bases, counts, offsets, block_m-padded offsets, the row-tile table and
//                     the -1 fill of padding rows (every step spread over the experts).
//   3. route_scatter: each chunk walks its pairs in flat order, 256 at a time; a pair's rank
//                     among equal keys inside its wavefront comes from 9 ballots (one per key
//                     bit), across wavefronts from LDS counts, so the placement is the stable
//                     order (ascending flat index inside each expert) bit for bit.
#include "afd_common.h"
#include "afd_internal.h"

namespace afd {

constexpr int kRouteThreads = 256;
constexpr int kScanThreads = 1024;
constexpr int kMaxChunks = 128;
constexpr int kKeyBits = 9;  // keys 0..256 (local expert, or num_local for "not local")
static_assert(kMaxChunks % (kScanThreads / kMaxLocalExperts) == 0, "chunk runs of the scan");

__device__ __forceinline__ int pair_key(int id, int e_lo, int num_local) {
  unsigned rel = static_cast<unsigned>(id - e_lo);
  return rel < static_cast<unsigned>(num_local) ? static_cast<int>(rel) : num_local;
}

__global__ __launch_bounds__(kRouteThreads) void route_hist_kernel(
    const int32_t* __restrict__ ids, int64_t pairs, int chunk, int e_lo, int num_local,
    int32_t* __restrict__ hist) {
  __shared__ int cnt[kMaxLocalExperts];
  for (int e = threadIdx.x; e < num_local; e += kRouteThreads) cnt[e] = 0;
  __syncthreads();
  const int64_t lo = int64_t(blockIdx.x) * chunk;
  const int64_t hi = lo + chunk < pairs ? lo + chunk : pairs;
  for (int64_t i = lo + threadIdx.x; i < hi; i += kRouteThreads) {
    int key = pair_key(ids[i], e_lo, num_local);
    if (key < num_local) atomicAdd(&cnt[key], 1);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < num_local; e += kRouteThreads)
    hist[int64_t(blockIdx.x) * num_local + e] = cnt[e];
}

__global__ __launch_bounds__(kScanThreads) void route_scan_kernel(
    int32_t* __restrict__ hist, int chunks, int num_local, int block_m,
    int32_t* __restrict__ counts, int32_t* __restrict__ offsets, int32_t* __restrict__ poff,
    int32_t* __restrict__ sorted_pairs, int32_t* __restrict__ tile_expert,
    int32_t* __restrict__ num_tiles) {
  __shared__ int part[kScanThreads];
  __shared__ int tot[kMaxLocalExperts];
  __shared__ int pof[kMaxLocalExperts + 1];
  const int t = threadIdx.x;
  // Expert e's chunks are split over G = kScanThreads / num_local threads (e, g); each loads
  // its contiguous run of at most kMaxPer chunks at once (independent loads, kept in
  // registers), the runs' bases come from the partial sums in LDS, then each thread rewrites
  // its chunks as exclusive bases without reloading them.
  constexpr int kMaxPer = kMaxChunks / (kScanThreads / kMaxLocalExperts);
  const int G = kScanThreads / num_local;
  const int per = (chunks + G - 1) / G;
  const int e = t % num_local, g = t / num_local;
  const bool active = g < G;
  const int c0 = active ? g * per : 0, c1 = active ? min(c0 + per, chunks) : 0;
  int hv[kMaxPer];
  int sum = 0;
#pragma unroll
  for (int k = 0; k < kMaxPer; ++k) {
    hv[k] = c0 + k < c1 ? hist[int64_t(c0 + k) * num_local + e] : 0;
    sum += hv[k];
  }
  part[t] = sum;
  __syncthreads();
  if (active) {
    int run = 0;
    for (int h = 0; h < g; ++h) run += part[h * num_local + e];
    if (g == 0) {
      int all = 0;
      for (int h = 0; h < G; ++h) all += part[h * num_local + e];
      tot[e] = all;
      counts[e] = all;
    }
#pragma unroll
    for (int k = 0; k < kMaxPer; ++k) {
      if (c0 + k < c1) hist[int64_t(c0 + k) * num_local + e] = run;
      run += hv[k];
    }
  }
  __syncthreads();
  // expert offsets and block_m-padded offsets: one wavefront, 4 experts per lane
  if (t < 64) {
    int o[4], q[4], so = 0, sp = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ex = t * 4 + i;
      const int c = ex < num_local ? tot[ex] : 0;
      o[i] = so;
      q[i] = sp;
      so += c;
      sp += (c + block_m - 1) / block_m * block_m;
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
        offsets[ex] = bo + o[i];
        poff[ex] = bp + q[i];
        pof[ex] = bp + q[i];
      }
    }
    if (t == 63) {
      offsets[num_local] = io;
      poff[num_local] = ip;
      pof[num_local] = ip;
      num_tiles[0] = ip / block_m;
    }
  }
  __syncthreads();
  // row-tile table (thread e writes expert e's tiles) and -1 on the padding rows of every
  // segment (the G threads of expert e stride over its at most block_m - 1 padding rows)
  if (t < num_local)
    for (int i = pof[t] / block_m, i1 = pof[t + 1] / block_m; i < i1; ++i) tile_expert[i] = t;
  if (active)
    for (int r = pof[e] + tot[e] + g; r < pof[e + 1]; r += G) sorted_pairs[r] = -1;
}

__global__ __launch_bounds__(kRouteThreads) void route_scatter_kernel(
    const int32_t* __restrict__ ids, int64_t pairs, int chunk, int e_lo, int num_local,
    const int32_t* __restrict__ hist, const int32_t* __restrict__ poff,
    int32_t* __restrict__ sorted_pairs, int32_t* __restrict__ pair_pos) {
  constexpr int kWaves = kRouteThreads / 64;
  __shared__ int run[kMaxLocalExperts + 1];
  __shared__ int wcnt[kWaves][kMaxLocalExperts + 1];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  for (int e = t; e < num_local; e += kRouteThreads)
    run[e] = poff[e] + hist[int64_t(blockIdx.x) * num_local + e];
  for (int i = t; i < kWaves * (kMaxLocalExperts + 1); i += kRouteThreads) (&wcnt[0][0])[i] = 0;
  __syncthreads();
  const int64_t lo = int64_t(blockIdx.x) * chunk;
  const int64_t hi = lo + chunk < pairs ? lo + chunk : pairs;
  const uint64_t below = (uint64_t(1) << lane) - 1;
  for (int64_t base = lo; base < hi; base += kRouteThreads) {
    const int64_t i = base + t;
    const bool live = i < hi;
    const int key = live ? pair_key(ids[i], e_lo, num_local) : num_local;
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

int launch_route(const int32_t* ids, int32_t n, const afd_moe_cfg& cfg, uint8_t* ws,
                 const afd_ws_layout& L, hipStream_t stream) {
  const int64_t pairs = int64_t(n) * cfg.topk;
  int chunks, chunk;
  route_chunking(pairs, &chunks, &chunk);
  int32_t* hist = reinterpret_cast<int32_t*>(ws + L.hist);
  int32_t* poff = reinterpret_cast<int32_t*>(ws + L.padded_offsets);
  int32_t* sorted = reinterpret_cast<int32_t*>(ws + L.sorted_pairs);
  int32_t* ppos = reinterpret_cast<int32_t*>(ws + L.pair_pos);
  if (chunks > 0) {
    hipLaunchKernelGGL(route_hist_kernel, dim3(chunks), dim3(kRouteThreads), 0, stream, ids,
                       pairs, chunk, cfg.expert_lo, cfg.num_local, hist);
    AFD_CHECK_LAUNCH();
  }
  hipLaunchKernelGGL(route_scan_kernel, dim3(1), dim3(kScanThreads), 0, stream, hist, chunks,
                     cfg.num_local, L.block_m, reinterpret_cast<int32_t*>(ws + L.counts),
                     reinterpret_cast<int32_t*>(ws + L.offsets), poff, sorted,
                     reinterpret_cast<int32_t*>(ws + L.tile_expert),
                     reinterpret_cast<int32_t*>(ws + L.num_tiles));
  AFD_CHECK_LAUNCH();
  if (chunks > 0) {
    hipLaunchKernelGGL(route_scatter_kernel, dim3(chunks), dim3(kRouteThreads), 0, stream, ids,
                       pairs, chunk, cfg.expert_lo, cfg.num_local, hist, poff, sorted, ppos);
    AFD_CHECK_LAUNCH();
  }
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
  return afd::launch_route(ids, n, *cfg, static_cast<uint8_t*>(ws), L,
                           static_cast<hipStream_t>(stream));
}
