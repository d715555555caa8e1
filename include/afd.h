/*
 * afd.h - C ABI of the MI355X (gfx950) F-side routed-expert path of an attention-FFN
 * disaggregated MoE deployment.
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t (as void*), only
 * enqueues work on that stream (no host synchronisation, no allocation, no global mutable
 * state besides the thread-local last HIP error) and returns 0 or a negative afd_status.
 *
 * Reference interfaces each group replaces (paths relative to the reference repository,
 * P = python/sgl_asap_plugin):
 *   afd_moe_ffn ................ the expert call FusedMoE(x, StandardTopKOutput(w, ids))
 *                                at P/srt/managers/scheduler.py:410-412 and its graph form
 *                                P/srt/model_executor/runner/ffn_cuda_graph_runner.py:60,65
 *   afd_route .................. the routing/permutation stage inside that call
 *                                (local_expert_offset / local_num_experts routing,
 *                                P/srt/layers/quantization/mxfp4_flashinfer_trtllm_moe.py:87-93)
 *   afd_quant_mxfp8 / _fp8_1x128 the activation quantizer quantize_routed_input
 *   / afd_quant_act              (mxfp4_flashinfer_trtllm_moe.py:59-61)
 *   afd_moe_ffn_job / .......... the graph runner's replay (P/srt/model_executor/runner/
 *   afd_job_set                  ffn_cuda_graph_runner.py:75-92) with the job read from a
 *                                device descriptor instead of copied into static inputs
 *   afd_moe_ffn_answer ......... the expert call followed by FfnServer.reply's done flag
 *                                (P/srt/managers/scheduler.py:410-412, P/transport/server.py
 *                                :340-350), the flag stored by the call's last workgroup
 *   afd_moe_ffn_q .............. the expert call on activations quantized before the arena
 *                                copy (the reference's TODO, scripts/run_asap.sh:110-111)
 *   afd_finalize ............... the finalize (top-k weighted sum, do_finalize=True,
 *                                mxfp4_flashinfer_trtllm_moe.py:97)
 *   afd_combine ................ AsapBuffer.recv's sum of partial outputs
 *                                (P/srt/layers/moe/token_dispatcher/asap.py:174-184) fused
 *                                with the shared-expert add (P/srt/batch_overlap/
 *                                operations_strategy.py:106-111)
 *   afd_silu_mul ............... the activation of the attention rank's shared-expert MLP
 *                                (computed at P/srt/batch_overlap/operations_strategy.py:94,
 *                                255 by SGLang's DeepseekV2MLP: SiluAndMul between its
 *                                gate_up and down projections)
 *   afd_pack_mxfp4 / _fp8_block  the quant methods' weight repack at load time
 *                                (FlashInfer layout, mxfp4_flashinfer_trtllm_moe.py:11-13)
 *   afd_repack_mxfp4 / ......... the checkpoint expert load (P/srt/model_loader/weight_utils.py
 *   _fp8_block                   :27-54 selects the tensors, SGLang's FusedMoE weight_loader
 *                                stores them; MXFP4 layout of P/srt/configs/model_config.py:3-7)
 *   afd_send ................... AttnChannel.send (P/transport/channel.py:317-362): the
 *                                backpressure waits, the payload copies to every F rank's
 *                                RecvArena region and the doorbells, as one call
 *   afd_reply .................. FfnServer.reply (P/transport/server.py:340-350): the
 *                                partial-sum copies and the done flags of a job, as one call
 *   afd_wait_replies ........... the reply waits of AttnChannel.wait (P/transport/channel.py
 *                                :364-377)
 *   afd_copy_async ............. cu.memcpy_async (P/transport/cuda_wrapper.py, used at
 *                                P/transport/channel.py:345-349, P/transport/server.py:347)
 *   afd_stream_write64 ......... cu.write64 / write32 (cuda_wrapper.py:258-270; doorbell at
 *                                channel.py:351-355, done flag at server.py:350)
 *   afd_stream_wait64 .......... cu.wait32 (cuda_wrapper.py:258-270; channel.py:339,370)
 *   afd_host_alloc / _free ..... the doorbell page of P/transport/memory.py:48-116
 *                                (pinned host memory on one GPU)
 */
#ifndef AFD_H_
#define AFD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AFD_ABI_VERSION 6

typedef void* afd_stream_t; /* a hipStream_t; NULL is the null stream */

/* Status codes. The Python layer maps them to the reference's exceptions. */
enum afd_status {
  AFD_OK = 0,
  AFD_ERR_ARG = -1,         /* null pointer or out-of-range argument (ValueError) */
  AFD_ERR_SHAPE = -2,       /* unsupported shape or alignment (ValueError) */
  AFD_ERR_UNSUPPORTED = -3, /* unsupported format or configuration (NotImplementedError) */
  AFD_ERR_HIP = -4,         /* a HIP call failed; afd_last_hip_error() has its hipError_t */
  AFD_ERR_WORKSPACE = -5    /* the workspace is smaller than afd_workspace_layout().total */
};

/* Expert weight formats. */
enum afd_weight_fmt {
  AFD_W_MXFP4 = 1,    /* E2M1 + UE8M0 per 32 along K; fp8 activations MXFP8 (e4m3 + UE8M0/32) */
  AFD_W_FP8_BLOCK = 2 /* e4m3 + fp32 per 128x128; fp8 activations e4m3 + fp32 per 1x128 */
};

/* Activation format of the expert GEMMs (the precision the MoE method runs its GEMMs in:
 * SGLang's MXFP4 method quantizes the input to MXFP8 under its default
 * flashinfer_mxfp4_moe_precision and has others, python/sgl_asap_plugin/srt/layers/
 * quantization/mxfp4_flashinfer_trtllm_moe.py:49-61; the reference also runs W4A16 experts,
 * MXFP4 weights with bf16 activations, through humming: scripts/run_ep.sh:4, README.md:25). */
enum afd_act_fmt {
  AFD_A_FP8 = 0, /* the weight format's fp8 activations (above): x and h are quantized */
  AFD_A_BF16 = 1 /* bf16 activations: x is read as it is, h is rounded to bf16, and the GEMMs
                    run on bf16 MFMA with the weights expanded to bf16 in registers (W4A16
                    for MXFP4 weights, W8A16 for FP8 blocks, whose fp32 block scales are
                    applied to the fp32 sums) */
};

/* Stream-wait conditions, as HIP's hipStreamWaitValue flags. */
enum afd_wait_cond { AFD_WAIT_GEQ = 0, AFD_WAIT_EQ = 1, AFD_WAIT_AND = 2, AFD_WAIT_NOR = 3 };

/* Activation of the gate_up output (FusedMoE's moe_runner_config.activation). */
enum afd_activation {
  AFD_ACT_SWIGLU = 0, /* h = silu(gate) * up ("silu") */
  AFD_ACT_SITU = 1,   /* h = L tanh(up / L) * A tanh(gate / A) * sigmoid(gate) ("situ"), with
                         A = act_alpha (SiTU's beta, FusedMoE gemm1_alpha) and L = act_limit
                         (its linear_beta, gemm1_clamp_limit): the function the reference's
                         SiTU hook runs, python/sgl_asap_plugin/srt/layers/quantization/
                         mxfp4_flashinfer_trtllm_moe.py:13-16 */
  AFD_ACT_SWIGLU_LIMIT = 2 /* h = silu(min(gate, L)) * clamp(up, -L, L), L = act_limit: SwiGLU
                              with DeepSeek-V4's swiglu_limit, which the reference hands to
                              FusedMoE (python/sgl_asap_plugin/srt/models/deepseek_v4.py:63) */
};

/* How the persistent GEMMs of the expert call hand out their output tiles. */
enum afd_tile_walk {
  AFD_WALK_STATIC = 0, /* a fixed share per workgroup: best when the call has the GPU's CUs to
                          itself */
  AFD_WALK_DYNAMIC = 1 /* taken in order from a per-XCD counter: when kernels of other
                          streams or parked stream waits (HIP runs hipStreamWaitValue as a
                          kernel) may hold CUs, a workgroup that starts late takes fewer tiles
                          instead of adding a whole round (one parked wait slowed a static
                          16384-token call by 38%, a dynamic one by <2%; on an idle GPU the
                          counter costs 1-4%) */
};

/* Shape of one MoE layer on one F rank. Experts [expert_lo, expert_lo + num_local) are
 * local; top-k ids are global expert ids; pairs with other ids are skipped.
 * Limits: hidden a multiple of 256 up to 16384, inter a multiple of 128 up to 16384,
 * num_local <= 256, topk <= 32, n <= 131071. */
typedef struct afd_moe_cfg {
  int32_t hidden;
  int32_t inter;
  int32_t topk;
  int32_t expert_lo;
  int32_t num_local;
  int32_t weight_fmt; /* enum afd_weight_fmt */
  int32_t activation; /* enum afd_activation (0: SwiGLU) */
  float act_alpha;    /* SiTU: A > 0 (unused otherwise) */
  float act_limit;    /* SiTU, SwiGLU with limit: L > 0 and finite (unused for SwiGLU) */
  int32_t tile_walk;  /* enum afd_tile_walk (0: static) */
  int32_t act_fmt;    /* enum afd_act_fmt (0: fp8) */
} afd_moe_cfg;

/* Packed expert weights of one layer (device pointers), as afd_pack_* writes them.
 *  MXFP4: w13 / w2 are tile images, the LDS bytes of one 128-wide K stage of one 256-row
 *    tile followed by that tile's UE8M0 scales: [E][N/256][K/128][256 x 64 B | 256 x 4 B]
 *    (17408 bytes each; N = 2I, K = H for w13; N = H, K = I for w2). In a tile, 16-byte
 *    chunk c (32 e2m1 values, element 2i in the low nibble) of row n sits at byte
 *    n*64 + 16*(c ^ (((n >> 1) ^ (n >> 2)) & 3)); scale j of row n at 16384 + 4n + (2(j & 1) | (j >> 1)). w13 rows
 *    interleave gate and up in groups of 32 (physical row 64j+q is gate row 32j+q for
 *    q < 32, else up row 32j+q-32). s13 and s2 are not used (NULL).
 *  FP8_BLOCK: w13 / w2 are FP8 images, the e4m3 bytes of one 64-wide K stage of one 256-row
 *    tile: [E][N/256][K/64][256 x 64 B] (16384 bytes each), 16-byte chunk c (16 e4m3 values)
 *    of row n at byte n*64 + 16*(c ^ (((n >> 1) ^ (n >> 2)) & 3)) as in an MXFP4 tile;
 *    s13 f32 [E][2I/128][H/128], s2 f32 [E][H/128][I/128]. w13 rows interleave gate and up
 *    in groups of 32 as above, while s13 keeps logical block order (gate blocks, then up
 *    blocks). */
typedef struct afd_expert_weights {
  const void* w13;
  const void* s13;
  const void* w2;
  const void* s2;
} afd_expert_weights;

/* Byte offsets of the internal buffers of afd_moe_ffn's workspace for n tokens. */
typedef struct afd_ws_layout {
  uint64_t total;          /* bytes the workspace must have */
  uint64_t xq, xs;         /* quantized activations [n][H] and their scales (MXFP4: e4m3 and
                              UE8M0 per 32, the 4 of each 128-wide K stage in stage order;
                              FP8 block: e4m3 and f32 per 1x128); bf16 activations: xq holds
                              a batched call's bf16 rows [n][H], xs is empty */
  uint64_t counts;         /* i32 [E] pairs per local expert */
  uint64_t offsets;        /* i32 [E+1] exclusive prefix of counts */
  uint64_t padded_offsets; /* i32 [E+1] the same with every segment padded to block_m */
  uint64_t sorted_pairs;   /* i32 [np_max] flat pair index t*k+kk per padded row, -1 = pad */
  uint64_t pair_pos;       /* i32 [n*k] padded row of each pair, -1 = not local */
  uint64_t tile_expert;    /* i32 [max_tiles] local expert of each block_m row tile */
  uint64_t num_tiles;      /* i32 [1] row tiles in use */
  uint64_t hist;           /* i32 router scratch */
  uint64_t hq, hs;         /* intermediate activations and their scales (MXFP4: down A tile
                              images, scales inside, hs empty; FP8 block: FP8 images of 256
                              rows x 64 K [row tiles][I/64], hs f32 [row tiles][I/128][256];
                              bf16 activations: bf16 images of 128 rows x 128 K (MXFP4) or
                              64 K (FP8 block), hs empty) */
  uint64_t y;              /* bf16 [np_max][H] per-pair down outputs */
  int64_t np_max;          /* padded rows reserved: n*k + E*(block_m-1), rounded up */
  int32_t block_m;         /* row tile of the grouped GEMMs */
  int32_t max_tiles;
} afd_ws_layout;

int afd_abi_version(void);
const char* afd_status_string(int status);
int afd_last_hip_error(void); /* hipError_t of the last AFD_ERR_HIP on this thread */

int afd_workspace_layout(const afd_moe_cfg* cfg, int32_t n, afd_ws_layout* out);

/* ---- weight packing (load time) -------------------------------------------------------
 * w: fp32 [mats][rows][cols] logical weights (for gate_up = 1: rows = 2I = [gate; up]).
 * afd_pack_mxfp4 writes mats * rows * (cols/2 + cols/32) bytes of tile images to `out`;
 * afd_pack_fp8_block writes mats * rows * cols bytes of FP8 images to q and the fp32
 * 128x128 block scales [mats][rows/128][cols/128] (logical block order) to s. Rows a
 * multiple of 256, cols of 128. */
int afd_pack_mxfp4(const float* w, int64_t mats, int32_t rows, int32_t cols, int32_t gate_up,
                   uint8_t* out, afd_stream_t stream);
int afd_pack_fp8_block(const float* w, int64_t mats, int32_t rows, int32_t cols,
                       int32_t gate_up, uint8_t* q, float* s, afd_stream_t stream);

/* ---- checkpoint repack (load time): already-quantized experts, bytes moved unchanged -----
 * afd_repack_mxfp4: codes u8 [mats][rows][cols/2] int8-packed e2m1 (element 2i in the low
 * nibble) + scales u8 [mats][rows][cols/32] E8M0, the checkpoint layout -> the tile images
 * afd_pack_mxfp4 writes (same size, same limits), holding the checkpoint's codes and scales
 * exactly. afd_repack_fp8_block: codes e4m3 [mats][rows][cols] -> the FP8 images
 * afd_pack_fp8_block writes (with gate_up = 1 through the 32-row gate/up interleave; rows a
 * multiple of 256, cols of 128); the fp32 128x128 block scales keep their logical order and
 * are used as they are. Pointers 16-byte aligned. */
int afd_repack_mxfp4(const uint8_t* codes, const uint8_t* scales, int64_t mats, int32_t rows,
                     int32_t cols, int32_t gate_up, uint8_t* out, afd_stream_t stream);
int afd_repack_fp8_block(const uint8_t* q, int64_t mats, int32_t rows, int32_t cols,
                         int32_t gate_up, uint8_t* out, afd_stream_t stream);

/* ---- activation quantizers -------------------------------------------------------------
 * x: bf16 [rows][cols]. MXFP8: q e4m3 [rows][cols], s u8 [rows][cols/32].
 * FP8 1x128: q e4m3 [rows][cols], s f32 [rows][cols/128]. */
int afd_quant_mxfp8(const uint16_t* x, int64_t rows, int32_t cols, uint8_t* q, uint8_t* s,
                    afd_stream_t stream);
int afd_quant_fp8_1x128(const uint16_t* x, int64_t rows, int32_t cols, uint8_t* q, float* s,
                        afd_stream_t stream);

/* ---- routing ----------------------------------------------------------------------------
 * ids: i32 [n][k]. Writes counts, offsets, padded_offsets, sorted_pairs, pair_pos,
 * tile_expert and num_tiles at the offsets of `layout` inside ws (the layout of
 * afd_workspace_layout for this n). Pairs of one expert keep ascending flat index. */
int afd_route(const int32_t* ids, int32_t n, const afd_moe_cfg* cfg, void* ws,
              uint64_t ws_bytes, afd_stream_t stream);

/* ---- the expert call ---------------------------------------------------------------------
 * out[t] = bf16(sum over local pairs (t, kk), kk ascending, of w[t,kk] * y(t,kk)) with
 * y = W2_e . silu(Wg_e . x_t) * (Wu_e . x_t) under the format's quantizers; 0 for tokens
 * with no local pair. x bf16 [n][H], ids i32 [n][k], w f32 [n][k], out bf16 [n][H]. */
int afd_moe_ffn(const afd_moe_cfg* cfg, const afd_expert_weights* weights, const uint16_t* x,
                const int32_t* ids, const float* w, int32_t n, void* ws, uint64_t ws_bytes,
                uint16_t* out, afd_stream_t stream);

/* The expert call on activations already quantized by afd_quant_act (fp8 activations on
 * the wire: A quantizes before the arena copy, the arena carries xq and xs, F reads them in
 * place). Same output as afd_moe_ffn on the bf16 x that afd_quant_act was given, bit for bit.
 * A configuration with bf16 activations has no quantized form (AFD_ERR_UNSUPPORTED).
 * The activation format on the wire is the reference's TODO (scripts/run_asap.sh:110-111,
 * P/transport/layout.py:64 ACT_BYTES = 2). */
int afd_moe_ffn_q(const afd_moe_cfg* cfg, const afd_expert_weights* weights, const uint8_t* xq,
                  const void* xs, const int32_t* ids, const float* w, int32_t n, void* ws,
                  uint64_t ws_bytes, uint16_t* out, afd_stream_t stream);

/* The expert call of a served job with its reply folded in: afd_moe_ffn (x != NULL, xq = xs =
 * NULL) or afd_moe_ffn_q (x = NULL, xq / xs), writing out (normally the asking rank's result
 * segment), then *done := value, stored by the last workgroup of the call's final launch once
 * every output row is visible device-wide, with system-scope release (so a stream or a host
 * waiting on a host-memory *done sees the output). Replaces, for a job whose output lands in
 * place, the expert call at P/srt/managers/scheduler.py:410-412 followed by the done flag of
 * FfnServer.reply (P/transport/server.py:340-350), without the separate stream store. done:
 * 8-byte aligned, pinned host or device memory; with n = 0 it is a stream store. The call's
 * workspace must not be shared with a call on another stream that overlaps it. */
int afd_moe_ffn_answer(const afd_moe_cfg* cfg, const afd_expert_weights* weights,
                       const uint16_t* x, const uint8_t* xq, const void* xs, const int32_t* ids,
                       const float* w, int32_t n, void* ws, uint64_t ws_bytes, uint16_t* out,
                       uint64_t* done, uint64_t value, afd_stream_t stream);

/* One job of a batched expert call: x bf16 [n][H] (or x = NULL and the rows quantized by
 * afd_quant_act: xq e4m3 [n][H] and xs their scales), ids i32 [n][k], w f32 [n][k], out bf16
 * [n][H]; done: NULL, or an 8-byte aligned counter (pinned host or device memory) that the
 * call sets to `value` once this job's output rows are visible device-wide. */
#define AFD_MAX_BATCH 8
typedef struct afd_batch_job {
  const uint16_t* x;
  const uint8_t* xq;
  const void* xs;
  const int32_t* ids;
  const float* w;
  uint16_t* out;
  uint64_t* done;
  uint64_t value;
  int32_t n;
  int32_t reserved; /* 0 */
} afd_batch_job;

/* One expert call over up to AFD_MAX_BATCH jobs of the same layer, as if their tokens were
 * one job: the routing, both GEMMs and the finalize run once over the concatenated tokens
 * (each expert's weights stream once for all the jobs, and its rows from different jobs share
 * row tiles), while every job reads its own x, ids and w and gets its own out. Each job's out
 * equals afd_moe_ffn (or, for quantized rows, afd_moe_ffn_q) on that job alone, bit for bit
 * (a token's output depends on its own row only). Every job gives its rows in the same form;
 * quantized rows are first copied into the workspace's activation buffers (device-to-device,
 * on `stream`). ws_bytes from afd_workspace_layout(cfg, sum of n), at most 131071 tokens. If
 * any job has a done counter, every job's counter is stored by the last workgroup of the
 * call's final launch (as afd_moe_ffn_answer does), after all the jobs' rows are visible.
 * Extends the FFN rank's per-job expert call (P/srt/managers/scheduler.py:410-412), which
 * concatenates the rows of one job's A ranks, to jobs of several replicas and slots that are
 * pending together. */
int afd_moe_ffn_batch(const afd_moe_cfg* cfg, const afd_expert_weights* weights,
                      const afd_batch_job* jobs, int32_t num_jobs, void* ws, uint64_t ws_bytes,
                      afd_stream_t stream);

/* The expert call without a workspace argument, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference. Same arguments and results as afd_moe_ffn,
 * bit for bit; the workspace is the library's own file-scope device array of
 * AFD_NOALLOC_SCRATCH_BYTES (128 MiB), one per GPU, held from the library's load until the
 * process ends. Jobs whose afd_workspace_layout(cfg, n).total exceeds it are rejected with
 * AFD_ERR_WORKSPACE (DeepSeek-V4 F-rank shape, hidden 4096 / inter 2048 / 64 local experts /
 * top-8: up to 568 tokens). Allocates nothing. Every call on a GPU uses that GPU's one array:
 * calls that overlap on one GPU (different streams, or host threads) race. */
#define AFD_NOALLOC_SCRATCH_BYTES (128ull << 20)
int afd_moe_ffn_noalloc(const afd_moe_cfg* cfg, const afd_expert_weights* weights,
                        const uint16_t* x, const int32_t* ids, const float* w, int32_t n,
                        uint16_t* out, afd_stream_t stream);

/* A job described in device memory, for callers that replay captured HIP graphs: the
 * launches of afd_moe_ffn_job read the descriptor when they run, so one capture serves every
 * job written into the descriptor afterwards (no copies into static buffers, no padding of
 * the job to the captured size). x: bf16 [n][H], or NULL with xq / xs as afd_quant_act
 * writes them; ids i32 [n][k]; w f32 [n][k]; out bf16 [n][H]. */
typedef struct afd_job {
  const uint16_t* x;
  const uint8_t* xq;
  const void* xs;
  const int32_t* ids;
  const float* w;
  uint16_t* out;
  int64_t n;
} afd_job;

/* The expert call on the job that `job` (device memory) holds when the launches run, with
 * n_cap the largest n it will hold: grids and the workspace are sized for n_cap (ws_bytes from
 * afd_workspace_layout(cfg, n_cap)); a descriptor n outside [0, n_cap] is clamped into it.
 * quantized = 0 reads job->x, 1 reads job->xq / job->xs. Results equal afd_moe_ffn's (or
 * afd_moe_ffn_q's) on the same job, bit for bit. Replaces the copy-in / pad / replay / copy-out
 * of the FFN rank's graph runner (P/srt/model_executor/runner/ffn_cuda_graph_runner.py:75-92). */
int afd_moe_ffn_job(const afd_moe_cfg* cfg, const afd_expert_weights* weights,
                    const afd_job* job, int32_t n_cap, int32_t quantized, void* ws,
                    uint64_t ws_bytes, afd_stream_t stream);

/* Enqueue on `stream` a write of *value (read now, on the host) into the device descriptor
 * `job`: ordered with the stream's launches, so a graph replayed after it sees the new job. */
int afd_job_set(afd_job* job, const afd_job* value, afd_stream_t stream);

/* The activation quantizer of the expert call (quantize_routed_input,
 * mxfp4_flashinfer_trtllm_moe.py:59-61) on its own: x bf16 [n][H] -> q e4m3 [n][H] and s:
 * MXFP4 weights: u8 [n][H/32] UE8M0, the 4 of each 128-wide K stage as blocks 0, 2, 1, 3
 * (block j at byte 2(j & 1) | (j >> 1) of its group); FP8 block weights: f32 [n][H/128].
 * Bf16 activations are not quantized (AFD_ERR_UNSUPPORTED). */
int afd_quant_act(const afd_moe_cfg* cfg, const uint16_t* x, int32_t n, uint8_t* q, void* s,
                  afd_stream_t stream);

/* afd_moe_ffn with hipEvent_t handles recorded on `stream` around its stages:
 * stage_events[0] before routing, [1] after the launch that histograms the pairs and
 * quantizes the activations, [2] after the router's scan and scatter, [3] after gate_up,
 * [4] after down, [5] after finalize. NULL entries are skipped.
 * Same replaced interface as afd_moe_ffn; for the per-stage timing of JobTimer
 * (P/srt/managers/scheduler.py:109-159). */
int afd_moe_ffn_profiled(const afd_moe_cfg* cfg, const afd_expert_weights* weights,
                         const uint16_t* x, const int32_t* ids, const float* w, int32_t n,
                         void* ws, uint64_t ws_bytes, uint16_t* out, afd_stream_t stream,
                         void* const* stage_events);

/* out[t] = bf16(sum_kk fp32(w[t,kk]) * fp32(y[pair_pos[t*k+kk]])) over pair_pos >= 0, each
 * product and each sum rounded to fp32 separately, kk ascending. */
int afd_finalize(const uint16_t* y, const int32_t* pair_pos, const float* w, int32_t n,
                 int32_t k, int32_t hidden, uint16_t* out, afd_stream_t stream);

/* A-side combine over num_parts (1..16) bf16 partial sums of numel elements:
 * routed = bf16(sum_f fp32(part_f)) (a copy for one part); out = shared ? bf16(fp32(routed)
 * + fp32(shared)) : routed. `parts` is a host array of device pointers. */
int afd_combine(const uint16_t* const* parts, int32_t num_parts, const uint16_t* shared,
                uint16_t* out, int64_t numel, afd_stream_t stream);

/* The shared-expert MLP's activation (replaces SGLang's SiluAndMul in the MLP the reference
 * calls at P/srt/batch_overlap/operations_strategy.py:94, 255): gate_up bf16 [n][2 inter]
 * (gate columns first, then up) -> out bf16 [n][inter], out = bf16(silu(g) * u) computed in
 * float with one rounding, silu(g) = g / (1 + e^-g). inter a multiple of 8, both pointers
 * 16-byte aligned, n * inter / 8 < 2^31. */
int afd_silu_mul(const uint16_t* gate_up, int64_t n, int32_t inter, uint16_t* out,
                 afd_stream_t stream);

/* ---- transport (one GPU: producer and consumer streams) ---------------------------------
 * Done flags are 64-bit message counters that only grow (a message's counter is the count of
 * messages sent on its slot, starting from the channel's base): afd_send's backpressure and
 * afd_wait_replies wait for counter >= value, so a later count, or a watchdog's release,
 * satisfies every earlier wait. Doorbell words carry the low 32 bits of the count in their
 * sequence field (the reference's bit layout, P/transport/layout.py:50-53). */
#define AFD_MAX_F 16

/* One message of an attention rank to every F rank (replaces AttnChannel.send,
 * P/transport/channel.py:317-362). On `stream`, in this order:
 *   1. for every F rank f with done[f] != NULL: wait until *done[f] >= done_min;
 *   2. the device-to-device copies of x (x_bytes), xs (xs_bytes, fp8 activations on the wire;
 *      NULL / 0 for bf16), ids and w (ids_bytes each) to region[f] + 0 / xs_off / ids_off / w_off
 *      for every f;
 *   3. for every f: the 64-bit store word[f] -> *bell[f].
 * Fields must not overlap inside a region; bell and done addresses 8-byte aligned. */
typedef struct afd_send_desc {
  int32_t num_f; /* 1..AFD_MAX_F */
  int32_t reserved;
  const void* x;
  uint64_t x_bytes;
  const void* xs;
  uint64_t xs_bytes;
  const void* ids;
  const void* w;
  uint64_t ids_bytes;
  uint64_t xs_off, ids_off, w_off;
  uint64_t done_min;
  void* region[AFD_MAX_F];
  uint64_t* bell[AFD_MAX_F];
  uint64_t word[AFD_MAX_F];
  uint64_t* done[AFD_MAX_F];
} afd_send_desc;
int afd_send(const afd_send_desc* msg, afd_stream_t stream);

/* One F-rank answer per row of a job (replaces FfnServer.reply, P/transport/server.py
 * :340-350): the copy of every row's partial sum (src -> dst, bytes; none when src == dst or
 * bytes == 0), then the 64-bit store value -> *done per row. 1..64 rows. */
typedef struct afd_reply_desc {
  const void* src;
  void* dst;
  uint64_t bytes;
  uint64_t* done;
  uint64_t value;
} afd_reply_desc;
int afd_reply(const afd_reply_desc* rows, int32_t num_rows, afd_stream_t stream);

/* Park `stream` until *done[f] >= seq for f < num_f (the reply waits of AttnChannel.wait,
 * P/transport/channel.py:364-377). */
int afd_wait_replies(uint64_t* const* done, int32_t num_f, uint64_t seq, afd_stream_t stream);

/* ---- transport primitives ---------------------------------------------------------------- */
int afd_host_alloc(void** ptr, uint64_t bytes); /* pinned, coherent, zero-filled */
int afd_host_free(void* ptr);
int afd_copy_async(void* dst, const void* src, uint64_t bytes, afd_stream_t stream);
int afd_stream_write64(afd_stream_t stream, uint64_t* addr, uint64_t value);
int afd_stream_wait64(afd_stream_t stream, uint64_t* addr, uint64_t value, uint64_t mask,
                      int32_t cond);

#ifdef __cplusplus
}
#endif

#endif /* AFD_H_ */
