// The expert call of one job on one F rank (afd_moe_ffn), its workspace layout, the
// finalize (top-k weighted sum) and the A-side combine.
//
//   (route histogram || quant x) -> route scatter -> grouped gate_up (+SwiGLU, +h quant)
//   -> grouped down -> finalize
//
// finalize and combine are HBM-bound gathers with fixed summation order, so their results
// are reproducible bit for bit (no atomics).
#include <cmath>
#include <mutex>
#include <vector>

#include "afd_common.h"
#include "afd_internal.h"

namespace afd {

static thread_local int g_last_hip_error = 0;

int set_hip_error(hipError_t e) {
  g_last_hip_error = static_cast<int>(e);
  return AFD_ERR_HIP;
}

int device_cu_count() {
  static std::mutex mu;
  static std::vector<int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if (dev >= static_cast<int>(cache.size())) cache.resize(dev + 1, 0);
  if (cache[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    cache[dev] = cus;
  }
  return cache[dev];
}

static uint64_t align256(uint64_t v) { return (v + 255) & ~uint64_t(255); }

// ---------------------------------------------------------------- finalize
// 128 lanes per workgroup, each a 16-byte vector: a 2048-byte column block of one token row
// per item (measured 4.6% faster than 256 lanes on the DeepSeek-V4 F-rank layer, 2% on the
// FP8 layer; 512 lanes 7% slower)
constexpr int kFinThreads = 128;
constexpr int kFinElems = 8;  // bf16 per lane = one 16-byte vector

// One (token, column block) item: out_row[col .. col + 7] of the call's token tok, whose k
// weights are w_row. kWriteThrough: the 16 bytes go out with the system-scope cache bits,
// which write them through the L2 to memory, so they are visible device-wide once
// acknowledged.
template <bool kWriteThrough>
__device__ __forceinline__ void finalize_item(const uint16_t* __restrict__ y,
                                              const int32_t* __restrict__ pair_pos,
                                              const float* __restrict__ w_row,
                                              uint16_t* __restrict__ out_row, int64_t tok,
                                              int col, int k, int hidden) {
  // products and sums round separately: no contraction of w * y + acc into an fma
#pragma clang fp contract(off)
  float acc[kFinElems];
#pragma unroll
  for (int i = 0; i < kFinElems; ++i) acc[i] = 0.0f;
  // up to 8 pairs at a time: their positions, then their rows, are loaded together; the sum
  // still runs over kk in ascending order. y is read once, so its rows are loaded
  // non-temporally (measured 4% faster at 2 local pairs per token, 12% at 8; the same hint
  // on the streaming reads of the quantizer and the combine made those slower).
  constexpr int kBatch = 8;
  for (int k0 = 0; k0 < k; k0 += kBatch) {
    int pos[kBatch];
    float wk[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const bool in = k0 + j < k;
      pos[j] = in ? pair_pos[tok * k + k0 + j] : -1;
      wk[j] = in ? w_row[k0 + j] : 0.0f;
    }
    v4i raw[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j)
      raw[j] = pos[j] >= 0 ? __builtin_nontemporal_load(reinterpret_cast<const v4i*>(y + int64_t(pos[j]) * hidden + col))
                           : v4i{0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      if (pos[j] < 0) continue;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t u = static_cast<uint32_t>(raw[j][i]);
        const float p0 = wk[j] * __uint_as_float(u << 16);
        const float p1 = wk[j] * __uint_as_float(u & 0xffff0000u);
        acc[2 * i] = acc[2 * i] + p0;
        acc[2 * i + 1] = acc[2 * i + 1] + p1;
      }
    }
  }
  v4i o;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    o[i] = static_cast<int>(pk_bf16(acc[2 * i], acc[2 * i + 1]));
  if constexpr (kWriteThrough) {
    // one 16-byte vector store per lane (a wavefront writes 1 KiB of whole lines), with the
    // system-scope cache bits; the caller waits for its acknowledgement
    // (the s_nop: a store of more than 8 bytes reads its data registers a cycle late, a
    // hazard the compiler does not see in inline assembly)
    asm volatile("global_store_dwordx4 %0, %1, off sc0 sc1\n\ts_nop 0" ::"v"(out_row + col), "v"(o)
                 : "memory");
  } else {
    *reinterpret_cast<v4i*>(out_row + col) = o;
  }
}

// Workgroups stride over the job's (token, column block) items (one item each when the grid
// covers them; with a descriptor, items past the job's tokens are skipped). With a reply, the
// grid is a few workgroups per CU; their output stores write through to memory, and each
// workgroup, once all its stores are acknowledged, counts itself in its group's counter (one
// atomic per workgroup, no cache write-back), the last of each group counts the group in
// reply.arrive, and the last group's stores the reply value (system scope), so a stream
// waiting on *reply.done (host memory) runs after every output row is in memory.
template <bool kReply>
__global__ __launch_bounds__(kFinThreads) void finalize_kernel(
    const uint16_t* __restrict__ y, const int32_t* __restrict__ pair_pos, JobIn jin, int k,
    int hidden, int col_blocks, Reply reply) {
  const JobIn job = resolve_job(jin);
  const uint32_t items = static_cast<uint32_t>(job.n) * static_cast<uint32_t>(col_blocks);
  for (uint32_t item = blockIdx.x; item < items; item += gridDim.x) {
    const uint32_t tok = item / static_cast<uint32_t>(col_blocks);
    const int col = static_cast<int>((item - tok * col_blocks) * kFinThreads + threadIdx.x) * kFinElems;
    if (col < hidden)
      finalize_item<kReply>(y, pair_pos, job_w_row(job, tok, k), job_out_row(job, tok, hidden),
                            tok, col, k, hidden);
  }
  if constexpr (kReply) {
    wait_vmcnt<0>();  // this lane's output stores are acknowledged (written through)
    __syncthreads();  // and every lane's of the workgroup
    // workgroup b counts itself in group b % groups; the last of a group counts the group in
    // the call's arrive word, and the last group stores the reply
    const uint32_t groups = gridDim.x < kArriveGroups ? gridDim.x : kArriveGroups;
    const uint32_t g = blockIdx.x % groups, size = (gridDim.x - g + groups - 1) / groups;
    uint32_t* group = reply.arrive + (kArriveGroupWord0 - kArriveWord) + g * kArriveGroupStride;
    if (threadIdx.x == 0 &&
        __hip_atomic_fetch_add(group, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == size - 1 &&
        __hip_atomic_fetch_add(reply.arrive, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
            groups - 1) {
#pragma unroll
      for (int b = 0; b < kMaxBatch; ++b)
        if (b < reply.count && reply.done[b] != nullptr)
          __hip_atomic_store(reply.done[b], reply.value[b], __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_SYSTEM);
    }
  }
}

// one workgroup per (token, column block) of job.n tokens (with a descriptor: of n_cap, the
// ones past the job's tokens do nothing); with a reply, at most kReplyGroupsPerCu workgroups
// per CU (1024 lanes)
constexpr int kReplyGroupsPerCu = 8;
static int launch_finalize(const uint16_t* y, const int32_t* pair_pos, const JobIn& job,
                           int32_t k, int32_t hidden, const Reply& reply, hipStream_t stream) {
  if (job.n == 0) return AFD_OK;
  const int col_blocks = (hidden / kFinElems + kFinThreads - 1) / kFinThreads;
  const int64_t items = col_blocks * job.n;
  if (reply.count > 0) {
    const int64_t cap = int64_t(kReplyGroupsPerCu) * device_cu_count();
    hipLaunchKernelGGL(finalize_kernel<true>, dim3(static_cast<unsigned>(items < cap ? items : cap)),
                       dim3(kFinThreads), 0, stream, y, pair_pos, job, k, hidden, col_blocks,
                       reply);
  } else {
    hipLaunchKernelGGL(finalize_kernel<false>, dim3(static_cast<unsigned>(items)),
                       dim3(kFinThreads), 0, stream, y, pair_pos, job, k, hidden, col_blocks,
                       reply);
  }
  AFD_CHECK_LAUNCH();
  return AFD_OK;
}

// ---------------------------------------------------------------- combine
constexpr int kMaxParts = 16;
struct PartList {
  const uint16_t* p[kMaxParts];
};

__global__ __launch_bounds__(256) void combine_kernel(PartList parts, int num_parts,
                                                      const uint16_t* __restrict__ shared,
                                                      uint16_t* __restrict__ out,
                                                      int64_t vecs) {
  for (int64_t v = blockIdx.x * int64_t(256) + threadIdx.x; v < vecs;
       v += int64_t(gridDim.x) * 256) {
    v4i first = reinterpret_cast<const v4i*>(parts.p[0])[v];
    v4i res;
    if (num_parts == 1) {
      res = first;
    } else {
      float acc[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t u = static_cast<uint32_t>(first[i]);
        acc[2 * i] = __uint_as_float(u << 16);
        acc[2 * i + 1] = __uint_as_float(u & 0xffff0000u);
      }
      for (int f = 1; f < num_parts; ++f) {
        v4i r = reinterpret_cast<const v4i*>(parts.p[f])[v];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          uint32_t u = static_cast<uint32_t>(r[i]);
          acc[2 * i] = __fadd_rn(acc[2 * i], __uint_as_float(u << 16));
          acc[2 * i + 1] = __fadd_rn(acc[2 * i + 1], __uint_as_float(u & 0xffff0000u));
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
        res[i] = static_cast<int>(uint32_t(f32_to_bf16(acc[2 * i])) |
                                  (uint32_t(f32_to_bf16(acc[2 * i + 1])) << 16));
    }
    if (shared) {
      v4i s = reinterpret_cast<const v4i*>(shared)[v];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t a = static_cast<uint32_t>(res[i]), b = static_cast<uint32_t>(s[i]);
        float lo = __fadd_rn(__uint_as_float(a << 16), __uint_as_float(b << 16));
        float hi = __fadd_rn(__uint_as_float(a & 0xffff0000u), __uint_as_float(b & 0xffff0000u));
        res[i] = static_cast<int>(uint32_t(f32_to_bf16(lo)) | (uint32_t(f32_to_bf16(hi)) << 16));
      }
    }
    reinterpret_cast<v4i*>(out)[v] = res;
  }
}

// ---------------------------------------------------------------- shared-expert activation
// h = bf16(silu(g) * u) for the rows of [gate | up] (bf16 [n][2 inter]): a lane takes 8
// columns, 16 bytes of g and 16 of u from one row, computes the routed experts' SwiGLU in
// float and rounds once. HBM-bound: per element 4 B read, 2 B written.
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* __restrict__ gu,
                                                       uint32_t vecs, uint32_t vpr,
                                                       uint16_t* __restrict__ out) {
  for (uint32_t v = blockIdx.x * 256u + threadIdx.x; v < vecs; v += gridDim.x * 256u) {
    const uint32_t r = v / vpr, c = v - r * vpr;
    const v4i* row = reinterpret_cast<const v4i*>(gu + int64_t(r) * vpr * 16);
    const v4i g = row[c], u = row[vpr + c];
    v4i o;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t a = static_cast<uint32_t>(g[i]), b = static_cast<uint32_t>(u[i]);
      o[i] = static_cast<int>(
          pk_bf16(act_swiglu(__uint_as_float(a << 16), __uint_as_float(b << 16)),
                  act_swiglu(__uint_as_float(a & 0xffff0000u), __uint_as_float(b & 0xffff0000u))));
    }
    reinterpret_cast<v4i*>(out + int64_t(r) * vpr * 8)[c] = o;
  }
}

// ---------------------------------------------------------------- configuration checks
static int check_cfg(const afd_moe_cfg* cfg) {
  if (!cfg) return AFD_ERR_ARG;
  if (cfg->topk < 1 || cfg->topk > kMaxTopk || cfg->num_local < 1 ||
      cfg->num_local > kMaxLocalExperts || cfg->expert_lo < 0)
    return AFD_ERR_ARG;
  if (cfg->hidden <= 0 || cfg->inter <= 0 || cfg->hidden % 256 || cfg->inter % 128 ||
      cfg->hidden > kMaxHidden || cfg->inter > kMaxInter)
    return AFD_ERR_SHAPE;
  if (cfg->weight_fmt != AFD_W_MXFP4 && cfg->weight_fmt != AFD_W_FP8_BLOCK)
    return AFD_ERR_UNSUPPORTED;
  if (cfg->activation != AFD_ACT_SWIGLU && cfg->activation != AFD_ACT_SITU &&
      cfg->activation != AFD_ACT_SWIGLU_LIMIT)
    return AFD_ERR_UNSUPPORTED;
  // SiTU's two constants are positive and finite (the reference raises ValueError without them)
  if (cfg->activation == AFD_ACT_SITU &&
      !(cfg->act_alpha > 0.0f && cfg->act_alpha < INFINITY && cfg->act_limit > 0.0f &&
        cfg->act_limit < INFINITY))
    return AFD_ERR_ARG;
  if (cfg->activation == AFD_ACT_SWIGLU_LIMIT && !(cfg->act_limit > 0.0f && cfg->act_limit < INFINITY))
    return AFD_ERR_ARG;
  if (cfg->tile_walk != AFD_WALK_STATIC && cfg->tile_walk != AFD_WALK_DYNAMIC) return AFD_ERR_ARG;
  if (cfg->act_fmt != AFD_A_FP8 && cfg->act_fmt != AFD_A_BF16) return AFD_ERR_UNSUPPORTED;
  return AFD_OK;
}

static bool bf16_act(const afd_moe_cfg& cfg) { return cfg.act_fmt == AFD_A_BF16; }

}  // namespace afd

using namespace afd;

extern "C" int afd_abi_version(void) { return AFD_ABI_VERSION; }

extern "C" const char* afd_status_string(int status) {
  switch (status) {
    case AFD_OK: return "ok";
    case AFD_ERR_ARG: return "invalid argument";
    case AFD_ERR_SHAPE: return "unsupported shape or alignment";
    case AFD_ERR_UNSUPPORTED: return "unsupported format or configuration";
    case AFD_ERR_HIP: return "HIP runtime error";
    case AFD_ERR_WORKSPACE: return "workspace too small";
    default: return "unknown status";
  }
}

extern "C" int afd_last_hip_error(void) { return g_last_hip_error; }

extern "C" int afd_workspace_layout(const afd_moe_cfg* cfg, int32_t n, afd_ws_layout* out) {
  int st = check_cfg(cfg);
  if (st != AFD_OK) return st;
  if (!out || n < 0 || n > 0x1ffff) return AFD_ERR_ARG;
  const int64_t H = cfg->hidden, I = cfg->inter, E = cfg->num_local;
  const int64_t pairs = int64_t(n) * cfg->topk;
  const bool mx = cfg->weight_fmt == AFD_W_MXFP4;
  const bool a16 = bf16_act(*cfg);
  const int64_t bm = block_m_of(*cfg);
  const int64_t np_max = (pairs + E * (bm - 1) + bm - 1) / bm * bm;
  uint64_t o = 0;
  auto take = [&](uint64_t bytes) {
    uint64_t at = o;
    o = align256(o + bytes);
    return at;
  };
  afd_ws_layout L;
  const uint64_t max_tiles = uint64_t(np_max / bm);
  // xq / xs: the per-token e4m3 rows and their scales (MXFP4: UE8M0 per 32, in stage order;
  // FP8 block: fp32 per 1x128). MXFP4: hq holds the down GEMM's A images (the h rows in
  // expert order, scales inside, hs empty); FP8 block: hq the down GEMM's FP8 A images (256
  // rows x 64 K) and hs their fp32 1x128 scales [row tiles][I/128][256]. bf16 activations: xq holds a batched call's bf16 rows (a single job's
  // are read in place), hq the down GEMM's bf16 A images (MXFP4: 32 KiB per 128 K, FP8 block:
  // 16 KiB per 64 K; the same bytes), xs and hs are empty.
  L.xq = take(a16 ? uint64_t(n) * H * 2 : uint64_t(n) * H);
  L.xs = take(a16 ? 0 : mx ? uint64_t(n) * (H / 32) : uint64_t(n) * (H / 128) * 4);
  L.counts = take(E * 4);
  L.offsets = take((E + 1) * 4);
  L.padded_offsets = take((E + 1) * 4);
  L.sorted_pairs = take(uint64_t(np_max) * 4);
  L.pair_pos = take(uint64_t(pairs) * 4);
  L.tile_expert = take(max_tiles * 4);
  L.num_tiles = take(kCallCounterBytes);  // num_tiles, then the call's counters
  L.hist = take(uint64_t(128) * E * 4);
  L.hq = take(a16  ? max_tiles * (I / kImgK) * kImgA16
               : mx ? max_tiles * (I / kImgK) * kImgA + kImgReadSlack
                    : uint64_t(np_max) * I);
  L.hs = take(mx || a16 ? 0 : uint64_t(np_max) * (I / 128) * 4);
  L.y = take(uint64_t(np_max) * H * 2);
  L.total = o;
  L.np_max = np_max;
  L.block_m = static_cast<int32_t>(bm);
  L.max_tiles = static_cast<int32_t>(max_tiles);
  *out = L;
  return AFD_OK;
}

// job: the job's pointers and n by value, or its descriptor with job.n = n_cap. quantized:
// the rows come quantized by afd_quant_act (xq / xs, or the descriptor's) instead of as bf16
// x, which is quantized here. With bf16 activations the GEMMs read bf16 rows: staged_x (a
// batch's rows, staged in the workspace) or else the job's x (or the descriptor's).
static int moe_ffn_impl(const afd_moe_cfg* cfg, const afd_expert_weights* weights,
                        const JobIn& job, bool quantized, const uint8_t* xq, const void* xs,
                        void* ws, uint64_t ws_bytes, afd_stream_t stream, void* const* ev,
                        const Reply* answer = nullptr, const uint16_t* staged_x = nullptr) {
  if (job.n < 0 || job.n > 0x1ffff) return AFD_ERR_ARG;
  const int32_t n = static_cast<int32_t>(job.n);
  afd_ws_layout L;
  int st = afd_workspace_layout(cfg, n, &L);
  if (st != AFD_OK) return st;
  const bool a16 = bf16_act(*cfg);
  if (a16 && quantized) return AFD_ERR_UNSUPPORTED;  // bf16 activations have no quantized form
  if (!weights || !weights->w13 || !weights->w2) return AFD_ERR_ARG;
  if (cfg->weight_fmt == AFD_W_FP8_BLOCK && (!weights->s13 || !weights->s2)) return AFD_ERR_ARG;
  const bool rows_ok = quantized ? (xq && xs) : job.x != nullptr;
  if (!job.desc && n > 0 && (!rows_ok || !job.ids || !job.w || !job.out)) return AFD_ERR_ARG;
  if (!ws) return AFD_ERR_ARG;
  if (ws_bytes < L.total) return AFD_ERR_WORKSPACE;
  // the gate_up GEMMs address token rows with 32-bit byte offsets
  if (uint64_t(n) * cfg->hidden * (a16 ? 2 : 1) > 0xffffffffull) return AFD_ERR_SHAPE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto mark = [&](int i) -> int {
    if (ev && ev[i]) AFD_CHECK_HIP(hipEventRecord(static_cast<hipEvent_t>(ev[i]), s));
    return AFD_OK;
  };
  if ((st = mark(0)) != AFD_OK) return st;
  if (n > 0) {
    uint8_t* wsb = static_cast<uint8_t*>(ws);
    const bool mx = cfg->weight_fmt == AFD_W_MXFP4;
    // routing and the activation quantization (one launch beside the expert histogram), then
    // the pair scatter; stage mark 1 falls between the two launches
    Reply reply = {};
    if (answer != nullptr) {
      reply = *answer;
      reply.arrive = call_counters(wsb, L) + kArriveWord;
    }
    st = launch_route_quant(job, !quantized && !a16, *cfg, wsb, L, s,
                            ev && ev[1] ? static_cast<hipEvent_t>(ev[1]) : nullptr);
    if (st != AFD_OK) return st;
    if ((st = mark(2)) != AFD_OK) return st;
    if (a16) {
      const uint16_t* rows = staged_x != nullptr ? staged_x : job.x;
      st = launch_a16_gate_up(*cfg, *weights, wsb, L, rows, staged_x ? nullptr : job.desc, s);
    } else {
      const uint8_t* aq = quantized ? xq : wsb + L.xq;
      const void* as = quantized ? xs : static_cast<const void*>(wsb + L.xs);
      const afd_job* rows_desc = quantized ? job.desc : nullptr;
      st = mx ? launch_mx_gate_up(*cfg, *weights, wsb, L, aq, as, rows_desc, s)
              : launch_fp8_gate_up(*cfg, *weights, wsb, L, aq, as, rows_desc, s);
    }
    if (st != AFD_OK || (st = mark(3)) != AFD_OK) return st;
    st = a16  ? launch_a16_down(*cfg, *weights, wsb, L, s)
         : mx ? launch_mx_down(*cfg, *weights, wsb, L, n, s)
              : launch_fp8_down(*cfg, *weights, wsb, L, n, s);
    if (st != AFD_OK || (st = mark(4)) != AFD_OK) return st;
    st = launch_finalize(reinterpret_cast<const uint16_t*>(wsb + L.y),
                         reinterpret_cast<const int32_t*>(wsb + L.pair_pos), job, cfg->topk,
                         cfg->hidden, reply, s);
    if (st != AFD_OK) return st;
  } else {
    for (int i = 1; i < 5; ++i)
      if ((st = mark(i)) != AFD_OK) return st;
    for (int b = 0; answer != nullptr && b < answer->count; ++b)
      if (answer->done[b]) AFD_CHECK_HIP(hipStreamWriteValue64(s, answer->done[b], answer->value[b], 0));
  }
  return mark(5);
}

extern "C" int afd_moe_ffn(const afd_moe_cfg* cfg, const afd_expert_weights* weights,
                           const uint16_t* x, const int32_t* ids, const float* w, int32_t n,
                           void* ws, uint64_t ws_bytes, uint16_t* out, afd_stream_t stream) {
  const JobIn job{nullptr, x, ids, w, out, n};
  return moe_ffn_impl(cfg, weights, job, false, nullptr, nullptr, ws, ws_bytes, stream, nullptr);
}

// ---------------------------------------------------------------- allocation-free call
// The workspace of afd_moe_ffn_noalloc: file-scope device memory, one copy per GPU. In host
// code the name `scratch` stands for a host-side shadow, not a device address, so host code
// never passes it to a kernel or a copy: it uses the address hipGetSymbolAddress returns,
// taken once per device with that device current and kept per device.
static __device__ __align__(256) uint8_t scratch[AFD_NOALLOC_SCRATCH_BYTES];

static int scratch_address(void** out) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static void* address[kMaxDevices] = {};
  int dev = 0;
  AFD_CHECK_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return AFD_ERR_ARG;
  std::lock_guard<std::mutex> lock(mu);
  if (address[dev] == nullptr) {
    void* p = nullptr;
    AFD_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (p == nullptr) return AFD_ERR_ARG;
    address[dev] = p;
  }
  *out = address[dev];
  return AFD_OK;
}

extern "C" int afd_moe_ffn_noalloc(const afd_moe_cfg* cfg, const afd_expert_weights* weights,
                                   const uint16_t* x, const int32_t* ids, const float* w,
                                   int32_t n, uint16_t* out, afd_stream_t stream) {
  afd_ws_layout L;
  int st = afd_workspace_layout(cfg, n, &L);
  if (st != AFD_OK) return st;
  if (L.total > AFD_NOALLOC_SCRATCH_BYTES) return AFD_ERR_WORKSPACE;
  void* ws = nullptr;
  if ((st = scratch_address(&ws)) != AFD_OK) return st;
  const JobIn job{nullptr, x, ids, w, out, n};
  return moe_ffn_impl(cfg, weights, job, false, nullptr, nullptr, ws, AFD_NOALLOC_SCRATCH_BYTES,
                      stream, nullptr);
}

extern "C" int afd_moe_ffn_q(const afd_moe_cfg* cfg, const afd_expert_weights* weights,
                             const uint8_t* xq, const void* xs, const int32_t* ids,
                             const float* w, int32_t n, void* ws, uint64_t ws_bytes,
                             uint16_t* out, afd_stream_t stream) {
  const JobIn job{nullptr, nullptr, ids, w, out, n};
  return moe_ffn_impl(cfg, weights, job, true, xq, xs, ws, ws_bytes, stream, nullptr);
}

extern "C" int afd_moe_ffn_answer(const afd_moe_cfg* cfg, const afd_expert_weights* weights,
                                  const uint16_t* x, const uint8_t* xq, const void* xs,
                                  const int32_t* ids, const float* w, int32_t n, void* ws,
                                  uint64_t ws_bytes, uint16_t* out, uint64_t* done,
                                  uint64_t value, afd_stream_t stream) {
  if (!done || (reinterpret_cast<uintptr_t>(done) & 7) != 0) return AFD_ERR_ARG;
  if ((x == nullptr) == (xq == nullptr)) return AFD_ERR_ARG;  // exactly one activation form
  const JobIn job{nullptr, x, ids, w, out, n};
  Reply answer = {};
  answer.done[0] = done;
  answer.value[0] = value;
  answer.count = 1;
  return moe_ffn_impl(cfg, weights, job, x == nullptr, xq, xs, ws, ws_bytes, stream, nullptr,
                      &answer);
}

extern "C" int afd_moe_ffn_batch(const afd_moe_cfg* cfg, const afd_expert_weights* weights,
                                 const afd_batch_job* jobs, int32_t num_jobs, void* ws,
                                 uint64_t ws_bytes, afd_stream_t stream) {
  if (!jobs || num_jobs < 1 || num_jobs > kMaxBatch) return AFD_ERR_ARG;
  JobIn job = {};
  Reply answer = {};
  int64_t total = 0;
  bool any_done = false;
  // every non-empty job gives x, or xq and xs, as the first non-empty one does (an empty job's
  // pointers may be null and say nothing)
  bool quantized = false;
  for (int b = 0; b < num_jobs; ++b)
    if (jobs[b].n > 0) {
      quantized = jobs[b].x == nullptr;
      break;
    }
  for (int b = 0; b < num_jobs; ++b) {
    const afd_batch_job& jb = jobs[b];
    if (jb.n < 0 || jb.reserved != 0) return AFD_ERR_ARG;
    const bool rows_ok = quantized ? (!jb.x && jb.xq && jb.xs) : (jb.x && !jb.xq && !jb.xs);
    if (jb.n > 0 && (!rows_ok || !jb.ids || !jb.w || !jb.out)) return AFD_ERR_ARG;
    if (jb.done && (reinterpret_cast<uintptr_t>(jb.done) & 7) != 0) return AFD_ERR_ARG;
    job.first[b] = static_cast<int32_t>(total);
    job.bx[b] = jb.x;
    job.bids[b] = jb.ids;
    job.bw[b] = jb.w;
    job.bout[b] = jb.out;
    answer.done[b] = jb.done;
    answer.value[b] = jb.value;
    any_done = any_done || jb.done != nullptr;
    total += jb.n;
    if (total > 0x1ffff) return AFD_ERR_ARG;
  }
  job.first[num_jobs] = static_cast<int32_t>(total);
  job.batch = num_jobs;
  job.n = total;
  // the first non-empty job's pointers also stand as the call's (moe_ffn_impl checks them)
  for (int b = 0; b < num_jobs; ++b)
    if (jobs[b].n > 0) {
      job.x = jobs[b].x;
      job.ids = jobs[b].ids;
      job.w = jobs[b].w;
      job.out = jobs[b].out;
      break;
    }
  answer.count = any_done ? num_jobs : 0;
  afd_ws_layout L;
  int st = afd_workspace_layout(cfg, static_cast<int32_t>(total), &L);
  if (st != AFD_OK) return st;
  const bool a16 = bf16_act(*cfg);
  if (!quantized && !a16)
    return moe_ffn_impl(cfg, weights, job, false, nullptr, nullptr, ws, ws_bytes, stream,
                        nullptr, any_done ? &answer : nullptr);
  if (quantized && a16) return AFD_ERR_UNSUPPORTED;
  if (!ws) return AFD_ERR_ARG;
  if (ws_bytes < L.total) return AFD_ERR_WORKSPACE;
  uint8_t* wsb = static_cast<uint8_t*>(ws);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (a16) {
    // bf16 rows of the GEMMs: staged one job after another into the workspace's xq, which the
    // gate_up GEMM then gathers from as one job's rows (the router, the finalize and the output
    // rows still go through each job's own ids, w and out)
    const uint64_t row = uint64_t(cfg->hidden) * 2;
    for (int b = 0; b < num_jobs; ++b) {
      const uint64_t n = static_cast<uint64_t>(jobs[b].n);
      if (n == 0) continue;
      AFD_CHECK_HIP(hipMemcpyAsync(wsb + L.xq + uint64_t(job.first[b]) * row, jobs[b].x, n * row,
                                   hipMemcpyDeviceToDevice, s));
    }
    return moe_ffn_impl(cfg, weights, job, false, nullptr, nullptr, ws, ws_bytes, stream, nullptr,
                        any_done ? &answer : nullptr, reinterpret_cast<const uint16_t*>(wsb + L.xq));
  }
  // quantized rows: staged one job after another into the workspace's xq / xs, which the
  // call then reads as one job's
  const uint64_t q_row = uint64_t(cfg->hidden);
  const uint64_t s_row = cfg->weight_fmt == AFD_W_MXFP4 ? uint64_t(cfg->hidden / 32)
                                                        : uint64_t(cfg->hidden / 128) * 4;
  for (int b = 0; b < num_jobs; ++b) {
    const uint64_t n = static_cast<uint64_t>(jobs[b].n);
    if (n == 0) continue;
    const uint64_t t0 = static_cast<uint64_t>(job.first[b]);
    AFD_CHECK_HIP(hipMemcpyAsync(wsb + L.xq + t0 * q_row, jobs[b].xq, n * q_row,
                                 hipMemcpyDeviceToDevice, s));
    AFD_CHECK_HIP(hipMemcpyAsync(wsb + L.xs + t0 * s_row, jobs[b].xs, n * s_row,
                                 hipMemcpyDeviceToDevice, s));
  }
  return moe_ffn_impl(cfg, weights, job, true, wsb + L.xq, wsb + L.xs, ws, ws_bytes, stream,
                      nullptr, any_done ? &answer : nullptr);
}

extern "C" int afd_moe_ffn_job(const afd_moe_cfg* cfg, const afd_expert_weights* weights,
                               const afd_job* job, int32_t n_cap, int32_t quantized, void* ws,
                               uint64_t ws_bytes, afd_stream_t stream) {
  if (!job) return AFD_ERR_ARG;
  const JobIn jin{job, nullptr, nullptr, nullptr, nullptr, n_cap};
  return moe_ffn_impl(cfg, weights, jin, quantized != 0, nullptr, nullptr, ws, ws_bytes, stream,
                      nullptr);
}

__global__ void job_set_kernel(afd_job* __restrict__ job, afd_job value) {
  if (threadIdx.x == 0) *job = value;
}

extern "C" int afd_job_set(afd_job* job, const afd_job* value, afd_stream_t stream) {
  if (!job || !value) return AFD_ERR_ARG;
  if ((reinterpret_cast<uintptr_t>(job) & 7) != 0) return AFD_ERR_ARG;
  hipLaunchKernelGGL(job_set_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), job,
                     *value);
  AFD_CHECK_LAUNCH();
  return AFD_OK;
}

extern "C" int afd_quant_act(const afd_moe_cfg* cfg, const uint16_t* x, int32_t n, uint8_t* q,
                             void* s, afd_stream_t stream) {
  int st = check_cfg(cfg);
  if (st != AFD_OK) return st;
  if (bf16_act(*cfg)) return AFD_ERR_UNSUPPORTED;  // bf16 activations are not quantized
  if (n < 0 || n > 0x1ffff) return AFD_ERR_ARG;
  if (n > 0 && (!x || !q || !s)) return AFD_ERR_ARG;
  return launch_quant_act(*cfg, x, n, q, s, static_cast<hipStream_t>(stream));
}

extern "C" int afd_moe_ffn_profiled(const afd_moe_cfg* cfg, const afd_expert_weights* weights,
                                    const uint16_t* x, const int32_t* ids, const float* w,
                                    int32_t n, void* ws, uint64_t ws_bytes, uint16_t* out,
                                    afd_stream_t stream, void* const* stage_events) {
  const JobIn job{nullptr, x, ids, w, out, n};
  return moe_ffn_impl(cfg, weights, job, false, nullptr, nullptr, ws, ws_bytes, stream,
                      stage_events);
}

extern "C" int afd_finalize(const uint16_t* y, const int32_t* pair_pos, const float* w,
                            int32_t n, int32_t k, int32_t hidden, uint16_t* out,
                            afd_stream_t stream) {
  if (n < 0 || k < 1 || k > kMaxTopk) return AFD_ERR_ARG;
  if (n > 0 && (!y || !pair_pos || !w || !out)) return AFD_ERR_ARG;
  if (hidden <= 0 || hidden % kFinElems) return AFD_ERR_SHAPE;
  const JobIn job{nullptr, nullptr, nullptr, w, out, n};
  return launch_finalize(y, pair_pos, job, k, hidden, Reply{}, static_cast<hipStream_t>(stream));
}

extern "C" int afd_silu_mul(const uint16_t* gate_up, int64_t n, int32_t inter, uint16_t* out,
                            afd_stream_t stream) {
  if (n < 0 || inter <= 0) return AFD_ERR_ARG;
  if (n == 0) return AFD_OK;
  if (!gate_up || !out) return AFD_ERR_ARG;
  if (inter % 8 || reinterpret_cast<uintptr_t>(gate_up) % 16 || reinterpret_cast<uintptr_t>(out) % 16)
    return AFD_ERR_SHAPE;
  // the kernel's 32-bit vector index must not wrap when it steps past the end
  const int64_t vecs = n * (inter / 8);
  if (vecs > 0x7fffffffll) return AFD_ERR_SHAPE;
  int64_t grid = (vecs + 255) / 256;
  if (grid > int64_t(8) * device_cu_count()) grid = int64_t(8) * device_cu_count();
  hipLaunchKernelGGL(silu_mul_kernel, dim3(static_cast<unsigned>(grid)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), gate_up, static_cast<uint32_t>(vecs),
                     static_cast<uint32_t>(inter / 8), out);
  AFD_CHECK_LAUNCH();
  return AFD_OK;
}

extern "C" int afd_combine(const uint16_t* const* parts, int32_t num_parts,
                           const uint16_t* shared, uint16_t* out, int64_t numel,
                           afd_stream_t stream) {
  if (!parts || !out || num_parts < 1 || num_parts > kMaxParts || numel < 0) return AFD_ERR_ARG;
  if (numel % 8) return AFD_ERR_SHAPE;
  PartList pl = {};
  for (int f = 0; f < num_parts; ++f) {
    if (!parts[f]) return AFD_ERR_ARG;
    pl.p[f] = parts[f];
  }
  if (numel == 0) return AFD_OK;
  const int64_t vecs = numel / 8;
  int64_t grid = (vecs + 255) / 256;
  if (grid > 4 * 2048) grid = 4 * 2048;
  hipLaunchKernelGGL(combine_kernel, dim3(static_cast<unsigned>(grid)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), pl, num_parts, shared, out, vecs);
  AFD_CHECK_LAUNCH();
  return AFD_OK;
}
