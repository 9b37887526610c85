/*
 * specmoe_mi355x.h -- C ABI of the MI355X (gfx950) MoE verify-step hot path.
 *
 * One shared library, libspecmoe_mi355x.so, built with hipcc --offload-arch=gfx950.
 * Every compute entry point (all but the host-memory and transfer-engine services at the
 * end, which allocate host memory and block the calling thread where stated):
 *   - takes plain device pointers and sizes (no framework types);
 *   - is stream-ordered on the hipStream_t passed as `stream` (NULL = default stream);
 *   - never synchronises the host and never allocates device memory: scratch space is the
 *     caller's `workspace` (size from smx_moe_workspace_size);
 *   - returns 0 on success, an SMX_ERR_* code (>= 1000) for a rejected argument, or the
 *     hipError_t of a failed launch. smx_error_string() names every code.
 * Calls are safe from several host threads on different streams with different workspaces.
 * The smx_set_* configuration functions are not: they set process-wide values that every
 * later call reads without synchronisation, so change them only while no MoE call is being
 * issued on another thread (the reference drives the MoE layer from one thread).
 *
 * Tensors are row-major and densely packed. Element types are SMX_F32 / SMX_F16 / SMX_BF16.
 *
 * Expert pool ("page") layout, one page per pool slot, page_elems = 3*I*H elements:
 *   [ W1 = gate (I x H) | W3 = up (I x H) | W2 = down (H x I) ]
 * (reference: specmoe/layers/FusedMoE.py:485-505, the weight_loader that packs it, and
 *  specmoe/layers/fused_moe_kernel.py:289-290, which derives I from the page size).
 */
#ifndef SPECMOE_MI355X_H
#define SPECMOE_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum smx_dtype { SMX_F32 = 0, SMX_F16 = 1, SMX_BF16 = 2 };

enum smx_status {
  SMX_OK = 0,
  SMX_ERR_INVALID_ARG = 1000,     /* null pointer, negative size, top_k > E, ... */
  SMX_ERR_UNSUPPORTED = 1001,     /* shape outside the kernels' limits (see below) */
  SMX_ERR_WORKSPACE = 1002,       /* workspace smaller than smx_moe_workspace_size() */
  SMX_ERR_MISALIGNED = 1003,      /* a tensor base is not 16-byte aligned */
  SMX_ERR_TIMEOUT = 1004,         /* smx_h2d_wait: the task did not finish in time */
  SMX_ERR_NOT_FOUND = 1005,       /* smx_h2d_wait: no such task id (or it was cleared) */
  SMX_ERR_SCRATCH = 1006          /* smx_fused_moe_forward_noalloc: sizes need more workspace
                                     than SMX_NOALLOC_SCRATCH_BYTES */
};

/* Limits: 1 <= E <= 256; 1 <= top_k <= min(E, 16); H and I multiples of 128 for 16-bit
 * types and of 64 for fp32 (a weight row is a whole number of 256-byte chunks); H, I <= 2^20;
 * page_elems <= 2^30 and page bytes < 2^32. Any T: a MoE call with more than 16384
 * assignments (T*top_k), or whose activations exceed 2^31 bytes, runs as consecutive passes
 * over token chunks on its stream (the expert sort holds 16384 assignments), sharing the
 * workspace, which the *_workspace_size queries size for the largest chunk.
 * T == 0 is a no-op. Shapes outside these limits return SMX_ERR_UNSUPPORTED. */

/* Library version (major*10000 + minor*100 + patch). */
int smx_version(void);

/* Human-readable name of a status code returned by any entry point. */
const char* smx_error_string(int code);

/*
 * Routing: fp32 softmax over E experts, then top_k rounds of arg-max (ties go to the lower
 * expert index), optional renormalisation w /= sum_j w.
 * Replaces sglang.srt.layers.moe.topk.select_experts(use_grouped_topk=False) as called at
 * specmoe/layers/FusedMoE.py:174-185 (sglang==0.4.5.post3, which dispatches to
 * sgl_kernel.topk_softmax and renormalises in torch).
 *   logits  [T, E] of logits_dtype
 *   topk_weights [T, top_k] fp32 out, topk_ids [T, top_k] int32 out (descending weight).
 */
int smx_topk_softmax(const void* logits, int logits_dtype, int64_t T, int64_t E,
                     int64_t top_k, int renormalize,
                     float* topk_weights, int32_t* topk_ids, void* stream);

/*
 * Grouped routing: the E experts form num_expert_group groups of gs = E / num_expert_group
 * consecutive experts, and only the topk_group best groups are selectable.
 *   correction_bias == NULL: scores s = the fp32 softmax of smx_topk_softmax (same bits);
 *     choice c = s; a group's score is the max of c over it.
 *   correction_bias [E] fp32: scores s = sigmoid(logit) (1/(1+exp(-x)) for x >= 0,
 *     e/(1+e) with e = exp(x) below); c = s + correction_bias; a group's score is the sum of
 *     its two largest c (needs gs >= 2).
 * Groups rank by descending score (ties to the lower group); the top_k selectable experts
 * by descending c (ties to the lower expert) are the picks, in that order; their weights are
 * s (not c), renormalised by the picks' sum when renormalize != 0. NaN ranks as -inf.
 * Replaces sglang.srt.layers.moe.topk.select_experts(use_grouped_topk=True) as called at
 * specmoe/layers/FusedMoE.py:174-185 (sglang==0.4.5.post3: grouped_topk without a bias,
 * biased_grouped_topk with one).
 *   logits [T, E] of logits_dtype; topk_weights [T, top_k] fp32 out, topk_ids [T, top_k]
 *   int32 out. Needs E % num_expert_group == 0, 1 <= topk_group <= num_expert_group and
 *   top_k <= topk_group * gs (SMX_ERR_INVALID_ARG otherwise); num_expert_group <= 64 (else
 *   SMX_ERR_UNSUPPORTED).
 */
int smx_grouped_topk(const void* logits, int logits_dtype, int64_t T, int64_t E, int64_t top_k,
                     int renormalize, int64_t num_expert_group, int64_t topk_group,
                     const float* correction_bias, float* topk_weights, int32_t* topk_ids,
                     void* stream);

/*
 * Token/expert alignment in the reference's padded format.
 * Replaces moe_align_block_size (specmoe/layers/fused_moe_kernel.py:16-85, which wraps
 * sgl_kernel.moe_align_block_size from sgl-kernel==0.1.2).
 *   topk_ids  [numel] int32, values in [0, E)
 *   sorted_ids  [numel + E*(block_size-1)] int32 out: for each expert in ascending order, the
 *               flat indices f (ascending) routed to it, then padding up to a multiple of
 *               block_size; every padding slot holds the sentinel `numel`.
 *   expert_ids  [ceil_div(numel + E*(block_size-1), block_size)] int32 out: the expert of each
 *               block; blocks at and past num_tokens_post_pad/block_size hold -1.
 *   num_tokens_post_pad [1] int32 out: sum over experts of round_up(count, block_size).
 */
int smx_moe_align_block_size(const int32_t* topk_ids, int64_t numel, int64_t E,
                             int64_t block_size, int32_t* sorted_ids, int32_t* expert_ids,
                             int32_t* num_tokens_post_pad, void* stream);

/* Bytes of workspace the two MoE entry points below need for these sizes. */
size_t smx_moe_workspace_size(int64_t T, int64_t H, int64_t I, int64_t E, int64_t top_k,
                              int dtype);

/*
 * The expert computation with routing already done:
 *   y[t] = sum_j w[t,j] * W2_e (silu(W1_e x[t]) * (W3_e x[t])),  e = topk_ids[t,j],
 * with the weights of expert e read from pool page expert_to_slot[e]. Intermediates are
 * rounded to `dtype` at the reference's points (gate/up outputs, silu*up, each weighted
 * down output, the final top_k sum); accumulation is fp32.
 * Replaces stack_fused_moe (specmoe/layers/fused_moe_kernel.py:253-349).
 *   hidden  [T, H] dtype;  out [T, H] dtype (may equal hidden: the in-place form)
 *   pool [num_slots, page_elems] dtype; expert_to_slot [E] int64 (device)
 *   topk_weights [T, top_k] fp32; topk_ids [T, top_k] int32 (device)
 * Only pool pages named by expert_to_slot[e] for routed experts e are read.
 * An id outside [0,E) or a slot outside [0,num_slots) contributes nothing to `out`.
 */
int smx_stack_fused_moe(const void* hidden, void* out, int dtype, int64_t T, int64_t H,
                        const void* pool, int64_t num_slots, int64_t page_elems,
                        const int64_t* expert_to_slot, int64_t E,
                        const float* topk_weights, const int32_t* topk_ids, int64_t top_k,
                        void* workspace, size_t workspace_bytes, void* stream);

/*
 * Routing plus expert computation in one call (smx_topk_softmax then smx_stack_fused_moe,
 * with the routing and expert sort fused into one launch).
 * Replaces FusedMoE.forward -> UnquantizedFusedMoEMethod.forward_cuda
 * (specmoe/layers/FusedMoE.py:508-532 and :155-196).
 *   router_logits [T, E] of logits_dtype.
 *   topk_weights_out / topk_ids_out: optional [T, top_k] outputs (NULL to skip).
 */
int smx_fused_moe_forward(const void* hidden, void* out, int dtype, int64_t T, int64_t H,
                          const void* router_logits, int logits_dtype, int64_t E,
                          int64_t top_k, int renormalize,
                          const void* pool, int64_t num_slots, int64_t page_elems,
                          const int64_t* expert_to_slot,
                          float* topk_weights_out, int32_t* topk_ids_out,
                          void* workspace, size_t workspace_bytes, void* stream);

/*
 * smx_fused_moe_forward without a workspace: the call allocates nothing. No counterpart in the
 * reference; it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).
 * The intermediates live in a device-resident scratch array of the library,
 * SMX_NOALLOC_SCRATCH_BYTES per GPU, which each GPU the library runs on holds from the
 * library's load until the process ends. Calls whose smx_moe_workspace_size() exceeds it return
 * SMX_ERR_SCRATCH before anything is launched (32 MiB holds every verify-step batch up to 128
 * tokens of the Mixtral-8x7B, Qwen1.5-MoE and DeepSeek-V2-Lite layer shapes).
 * Every call on one GPU shares that GPU's scratch and leaves its intermediates there: calls
 * that overlap on one GPU (two streams, or two threads without ordering) race. Nothing in the
 * scratch has to start at zero. Arguments and results otherwise as smx_fused_moe_forward, on the
 * device current at the call. The scratch's device address is looked up once per device, on
 * the first call there, and kept: resetting a device (hipDeviceReset) while the library is
 * loaded is not supported by this entry point.
 */
#define SMX_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int smx_fused_moe_forward_noalloc(const void* hidden, void* out, int dtype, int64_t T, int64_t H,
                                  const void* router_logits, int logits_dtype, int64_t E,
                                  int64_t top_k, int renormalize,
                                  const void* pool, int64_t num_slots, int64_t page_elems,
                                  const int64_t* expert_to_slot,
                                  float* topk_weights_out, int32_t* topk_ids_out, void* stream);

/* Bytes of workspace smx_fused_moe_shared_forward needs (shared_I = 0: no shared expert). */
size_t smx_moe_shared_workspace_size(int64_t T, int64_t H, int64_t I, int64_t E, int64_t top_k,
                                     int64_t shared_I, int dtype);

/*
 * A whole MoE block with an always-active shared expert, in one call:
 *   y[t] = round( round(routed[t] * routed_scaling_factor) + s[t] * shared[t] )
 *   routed[t] = round(sum_j round(w[t,j] * W2_e(...)))     as in smx_fused_moe_forward
 *   shared[t] = round(W2s (round(silu(round(W1s x[t])) * round(W3s x[t]))))
 *   s[t]      = round(sigmoid(shared_gate_logits[t])), or 1 when shared_gate_logits is NULL;
 *               the product s*shared is rounded, and every round() is to `dtype`.
 * This is the Qwen1.5-MoE / Qwen2-MoE block (gated shared expert, scale 1) and the
 * DeepSeek-V2 MoE block (ungated shared experts fused into one MLP of n_shared*I columns,
 * scaled routed output), with the rounding points of those blocks' unfused layers.
 * No counterpart in the reference: it serves no model with shared experts (its Mixtral
 * block is MixtralMoE.forward, specmoe/models/mixtral.py:106-115); the routed part is the
 * FusedMoE path above and the shared expert runs as one more expert in the same launches.
 *   shared_page [3*shared_I*H] of dtype, packed like a pool page: [W1s | W3s | W2s];
 *               NULL with shared_I = 0 for no shared expert.
 *   shared_gate_logits [T] of logits_dtype (the block's shared_expert_gate output) or NULL.
 * shared_I obeys the limits on I.
 */
int smx_fused_moe_shared_forward(const void* hidden, void* out, int dtype, int64_t T, int64_t H,
                                 const void* router_logits, int logits_dtype, int64_t E,
                                 int64_t top_k, int renormalize,
                                 const void* pool, int64_t num_slots, int64_t page_elems,
                                 const int64_t* expert_to_slot,
                                 const void* shared_page, int64_t shared_I,
                                 const void* shared_gate_logits, float routed_scaling_factor,
                                 float* topk_weights_out, int32_t* topk_ids_out,
                                 void* workspace, size_t workspace_bytes, void* stream);

/*
 * smx_fused_moe_shared_forward on routing the caller has done (topk_weights / topk_ids as
 * smx_stack_fused_moe takes them), for blocks whose routing is not the plain top-k softmax:
 * DeepSeek-V2's group-limited top-k and DeepSeek-V3's sigmoid top-k with a correction bias
 * (smx_grouped_topk). Same block arithmetic, workspace (smx_moe_shared_workspace_size) and
 * limits; shared_gate_logits [T] is of `dtype`. No counterpart in the reference (it serves no
 * model with shared experts); the routed part is smx_stack_fused_moe, which replaces
 * stack_fused_moe (specmoe/layers/fused_moe_kernel.py:253-349).
 */
int smx_stack_fused_moe_shared(const void* hidden, void* out, int dtype, int64_t T, int64_t H,
                               const void* pool, int64_t num_slots, int64_t page_elems,
                               const int64_t* expert_to_slot, int64_t E,
                               const float* topk_weights, const int32_t* topk_ids, int64_t top_k,
                               const void* shared_page, int64_t shared_I,
                               const void* shared_gate_logits, float routed_scaling_factor,
                               void* workspace, size_t workspace_bytes, void* stream);

/*
 * Post-attention residual add + RMSNorm + router gate in one kernel (one workgroup per token):
 *   s = hidden + residual (fp32; residual == NULL: s = hidden)
 *   residual      = round(s)                                      (in place, when given)
 *   normed_out    = round(s * (1 / sqrt(mean(s^2) + eps)) * norm_weight)   (may == hidden)
 *   router_logits = round(normed_out . gate_weight^T)   [T, E] of dtype, fp32 accumulation
 * gate_weight NULL: norm only (E and router_logits ignored).
 * Replaces RMSNorm.forward with a residual (specmoe/layers/layernorm.py:23-52; sglang's
 * fused_add_rmsnorm at :31) followed by MixtralMoE's router gate (specmoe/models/mixtral.py:
 * 84-91, 111), as called at specmoe/models/mixtral.py:310-313.
 * Limits: H * element size a multiple of 16 bytes, H <= 16384, E <= 256.
 */
int smx_add_rmsnorm_gate(const void* hidden, void* residual, void* normed_out, int dtype,
                         int64_t T, int64_t H, const void* norm_weight, float eps,
                         const void* gate_weight, int64_t E, void* router_logits, void* stream);

/* Bytes of workspace smx_moe_layer_forward needs. */
size_t smx_moe_layer_workspace_size(int64_t T, int64_t H, int64_t I, int64_t E, int64_t top_k,
                                    int64_t shared_I, int dtype);

/*
 * The post-attention half of a decoder layer in one call: smx_add_rmsnorm_gate (with the
 * token's top-k computed in the same kernel from the rounded logits) and then the MoE block
 * on the normalized states, written back into `hidden`:
 *   residual <- round(hidden + residual);  x = RMSNorm(...);  hidden <- MoE(x)
 * where MoE is smx_fused_moe_forward, or smx_fused_moe_shared_forward's block form when
 * shared_I > 0 or routed_scaling_factor != 1 (shared_gate_weight [H] gives the shared-expert
 * gate logit as one more row of the router gate; NULL: ungated).
 * Replaces MixtralDecoderLayer's post-attention step (specmoe/models/mixtral.py:310-313:
 * post_attention_layernorm then block_sparse_moe -> MixtralMoE.forward :106-115 ->
 * FusedMoE.forward, specmoe/layers/FusedMoE.py:508-532).
 *   router_logits_out [T, E] dtype, topk_weights_out / topk_ids_out [T, top_k]: optional.
 */
int smx_moe_layer_forward(void* hidden, void* residual, int dtype, int64_t T, int64_t H,
                          const void* norm_weight, float eps, const void* gate_weight, int64_t E,
                          int64_t top_k, int renormalize,
                          const void* pool, int64_t num_slots, int64_t page_elems,
                          const int64_t* expert_to_slot,
                          const void* shared_page, int64_t shared_I,
                          const void* shared_gate_weight, float routed_scaling_factor,
                          void* router_logits_out, float* topk_weights_out, int32_t* topk_ids_out,
                          void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------------
 * Host memory and host -> device streaming of expert pages.
 * --------------------------------------------------------------------------------------- */

/* Pinned (page-locked, portable) host memory via hipHostMalloc; free with smx_host_free.
 * Replaces cuda_host_alloc / free_pinned_tensor (specmoe/backend/pin_memory_allocator.py:
 * 7-28, 62-65), which hard-code libcudart's cudaMallocHost / cudaFreeHost. */
int smx_host_alloc(size_t bytes, void** ptr);
int smx_host_free(void* ptr);

/* Transfer classes in priority order (most urgent first), as TransferTaskType /
 * TASK_PRIORITY_MAPPING (specmoe/backend/htod_transfer_engine.py:16-30). */
enum smx_h2d_type { SMX_H2D_HIDDEN = 1, SMX_H2D_KV_CACHE = 2, SMX_H2D_DRAFT_KV_CACHE = 3,
                    SMX_H2D_WEIGHT = 4 };

/*
 * Asynchronous host -> device copy engine: one worker thread, a priority queue of chunk
 * copies (class, then layer -- layer 0 last --, then chunk index, then submission order).
 * A task's `bytes` (whole elements of `elem_bytes`) are split into `num_chunks` chunks, the
 * first (elements % num_chunks) one element longer; each chunk is copied with hipMemcpyAsync
 * on `stream` and waited for before the next chunk starts, so urgent tasks overtake long
 * ones between chunks. smx_h2d_wait blocks until the task's last chunk has landed
 * (timeout_s < 0: no limit) and returns its copy status; for SMX_H2D_WEIGHT tasks `seconds`
 * receives the time from its first chunk's start to its last chunk's end (else -1).
 * smx_h2d_clear forgets a task id (chunks already queued still run); resubmitting an id
 * starts a new task. smx_h2d_set_enabled(0) pauses the worker between chunks.
 * Replaces HtoDTransferEngine (specmoe/backend/htod_transfer_engine.py:73-520: start/stop,
 * submit_weight_loading_task :297-308, _submit_chunked_task :321-369, wait_for_completion
 * :375-411, clear_condition :413-420, the worker :405-489) for the weight streaming driven at
 * specmoe/backend/execution_engine.py:143-154,549-588. Streams passed in must have the default
 * priority.
 */
typedef struct smx_h2d_engine smx_h2d_engine;
int smx_h2d_engine_create(smx_h2d_engine** engine);
int smx_h2d_engine_destroy(smx_h2d_engine* engine);
int smx_h2d_submit(smx_h2d_engine* engine, int task_type, const char* task_id, void* dst,
                   const void* src, size_t bytes, size_t elem_bytes, int64_t num_chunks,
                   int64_t layer_id, void* stream);
int smx_h2d_wait(smx_h2d_engine* engine, const char* task_id, double timeout_s, double* seconds);
int smx_h2d_has_task(smx_h2d_engine* engine, const char* task_id);
int smx_h2d_clear(smx_h2d_engine* engine, const char* task_id);
int smx_h2d_set_enabled(smx_h2d_engine* engine, int enabled);
int smx_h2d_pending(smx_h2d_engine* engine);

/*
 * Expert-kernel selection. A MoE call whose expected tokens per active expert -- T*top_k
 * divided by the experts expected to be active under uniform routing,
 * E*(1 - (1 - top_k/E)^T) -- is at least `tokens_per_expert` runs the tiled expert kernels
 * (MFMA output tiles of 128 tokens by 128 intermediate columns / 256 hidden rows, for
 * prefill-sized batches); below it, the weight-streaming kernels. 0 = always tiled,
 * INT64_MAX = never; a negative value restores the default (64). Both produce the same
 * routing and rounding points; only the fp32 summation order over K differs. The workspace
 * size depends on the choice, so query it after setting. Process-wide, not synchronised with
 * calls in flight on other threads.
 * Plays the role of the reference's per-call kernel configuration rule (T*top_k vs E picks
 * the Triton tile sizes, specmoe/layers/fused_moe_kernel.py:293-306).
 */
int smx_set_tiled_min_tokens(int64_t tokens_per_expert);
int64_t smx_tiled_min_tokens(void);

/*
 * Down projection fused with the top-k combine, for batches of a few tokens on the
 * weight-streaming path: one wave per hidden row streams that row of every active expert's W2
 * (and of the shared expert's) and writes the layer output directly, instead of the K-split
 * down kernel writing fp32 partials and a combine kernel summing them. Same rounding points
 * (each routed term rounded after its weight is applied, the fp32 sum over j in order, the
 * block form); only the fp32 summation order over K differs.
 * `tokens` = 0: never; 1..8: every batch of at most that many tokens (larger values are taken
 * as 8); negative (the default): batches of at most 8 tokens whose output rows each stream at
 * most 48 KB of weight rows, T * (top_k * ceil(I*eb / 1 KB) + ceil(Is*eb / 1 KB)) <= 48 (the
 * DeepSeek-V2-Lite and Qwen1.5-MoE blocks at one and two tokens). The workspace size depends on the
 * choice, so query it after setting. Process-wide, like smx_set_tiled_min_tokens.
 * Replaces the third and fourth steps of stack_fused_moe
 * (specmoe/layers/fused_moe_kernel.py:339-347: the W2 GEMM with MUL_ROUTED_WEIGHT, then
 * torch.sum over top_k into hidden_states) for such batches.
 */
int smx_set_fused_down_max_tokens(int64_t tokens);
int64_t smx_fused_down_max_tokens(void);

/*
 * fp32 runs only: with `on` set, the routed experts' GEMM outputs are rounded to fp16 where
 * the reference's Triton kernel stores them for fp32 inputs -- the gate and up projections
 * (C1) and each assignment's weighted down projection (C3); the SiLU*up activation and the
 * top-k sum stay fp32 (specmoe/layers/fused_moe_kernel.py:203,248: compute_type is fp16 unless
 * the input is bf16; :319-327 and :337 keep the intermediates in the input dtype). Off by
 * default (true fp32 throughout). Shared-expert blocks are not affected (the reference has
 * none). bf16/fp16 runs already round to their own dtype at these points. Process-wide.
 */
int smx_set_fp32_gemm_outputs_fp16(int on);
int smx_fp32_gemm_outputs_fp16(void);

/*
 * Batches on the weight-streaming path over E <= 64 experts route inside the gate/up launch:
 * each routed workgroup computes the routing of the whole batch into its LDS and one of them
 * writes the routing records and top-k results for the later kernels, bit for bit the routing
 * kernels' records.
 *   - one wave: T*top_k <= 64 assignments, every expert's tokens one pass (T <= 16 per token
 *     tile of the plan, at most two tiles), router logits (when given) in the activation dtype
 *     in at most four top-k passes of 64/G tokens;
 *   - four waves (top-k), one of them sorting: router logits for T <= 64 tokens of one pass,
 *     T*top_k <= 256, T*G <= 512; or given ids (smx_stack_fused_moe and the forward calls
 *     whose top-k is too large to repeat, which then launch smx_topk_softmax's kernel first)
 *     up to 768 assignments, experts over several token ranges included.
 * Larger batches launch the routing kernels. 0 launches them always; default 1. Process-wide.
 * Plays the role of the reference's separate select_experts and moe_align_block_size launches
 * (specmoe/layers/FusedMoE.py:174-185, specmoe/layers/fused_moe_kernel.py:329-330).
 */
int smx_set_routing_in_gateup(int on);
int smx_routing_in_gateup(void);

/*
 * Waves per workgroup of the weight-streaming gate/up kernel: 4, 2 or 1 (the kernel's work is
 * the same -- one wave per 16 intermediate rows of an expert; only the grouping of waves into
 * workgroups, and with it the grid, changes), or 0 (the default rule): 4, unless that grid
 * holds more workgroups than the chip's 256 CUs but fewer than 320 (some CUs would run two
 * while most run one), then 2; with 4, for batches of at most 32 tokens over hidden rows of at
 * most 4 KB, the default also splits each item's K walk between wave pairs (two weight tiles per
 * workgroup, the halves' fp32 sums added once before the SwiGLU: a different, fixed summation
 * order).
 * Applies to batches of at most 32 tokens; larger ones always use 4. Outputs are identical
 * for every setting 1, 2 and 4 (same per-wave K walk and rounding). Process-wide, like
 * smx_set_tiled_min_tokens. Part of the expert-kernel configuration that replaces the
 * reference's per-call Triton tile choice (specmoe/layers/fused_moe_kernel.py:293-306).
 */
int smx_set_gateup_waves(int waves);
int smx_gateup_waves(void);

/*
 * Gate/up grids of the weight-streaming path with more workgroups than the chip holds at once
 * (two per CU) run, with `on` (the default), as a grid of at most that many workgroups that each
 * walk several work items in turn: the routing done inside the launch (small batches) then runs
 * once per workgroup instead of once per item, and each later item starts with its weight
 * loads. 0 launches one workgroup per item. Outputs are identical either way (same items, same
 * per-wave K walk). Process-wide, like smx_set_tiled_min_tokens.
 * Part of the expert-kernel configuration that replaces the reference's per-call Triton grid
 * (specmoe/layers/fused_moe_kernel.py:293-306).
 */
int smx_set_gateup_item_walk(int on);
int smx_gateup_item_walk(void);

/*
 * Batches routed inside the gate/up launch by its multi-wave form (up to 256 assignments over
 * at most 64 experts, at most 32 tokens: every expert's tokens one range of one pass) number
 * their routed work items by expert rather than by the routing's ranges, so that each
 * workgroup knows its first item before routing the batch and issues that item's first weight
 * loads first. `on` (the default) does this where fewer than 1 in 20 experts are expected to
 * get no token (their workgroups' early loads are wasted); 0 numbers items by range. Outputs
 * are identical either way (same items' arithmetic, same K walk). Process-wide.
 * Part of the expert-kernel configuration that replaces the reference's per-call Triton grid
 * (specmoe/layers/fused_moe_kernel.py:293-306).
 */
int smx_set_gateup_expert_items(int on);
int smx_gateup_expert_items(void);

/*
 * One-token MoE calls in one launch. A call of one token whose down projection and combine run
 * as one kernel (smx_set_fused_down_max_tokens) and whose routing runs inside the gate/up launch
 * -- the DeepSeek-V2-Lite and Qwen1.5-MoE blocks at one token -- runs, with `on`, as a single
 * launch: the gate/up workgroups, then in the same grid the fused down + combine
 * workgroups, which load their W2 rows while gate/up runs and wait inside the launch (bounded
 * in time) until every gate/up workgroup has stored its activation rows. Outputs are identical
 * to the two-launch form's. Not used while `stream` is capturing a graph (the two-launch form
 * runs instead). Off by default: on MI355X the two launches measured faster (DeepSeek-V2-Lite
 * block at one token: 31.1 vs 37.0 us per layer). Process-wide, like smx_set_tiled_min_tokens.
 * Replaces, at one token, the launch sequence of stack_fused_moe after routing -- the two
 * fused_moe_kernel GEMMs, silu_and_mul and the torch.sum combine
 * (specmoe/layers/fused_moe_kernel.py:329-347).
 */
int smx_set_single_launch_layer(int on);
int smx_single_launch_layer(void);

/*
 * Test hook of the single-launch form's in-launch wait. publish = 0: the gate/up workgroups do
 * not publish their activation rows, so every down workgroup gives up after wait_us
 * microseconds, writes NaN to its outputs and stores the call's value in the status word (the
 * workspace word after the flags: SMX_PLAN_SYNC_OFFSET); every workgroup still ends normally.
 * publish = 1 is normal operation. wait_us <= 0 restores the default bound (100 ms).
 * No counterpart in the reference: a failure-path test hook.
 */
int smx_set_layer_sync_test(int publish, int64_t wait_us);

/*
 * The launch plan a MoE call of these sizes takes under the current settings, on the host
 * only (no device work; usable without a GPU). Fills out[i] for i < min(n, SMX_PLAN_FIELDS)
 * in the order of enum smx_plan_field and returns SMX_PLAN_FIELDS, or an SMX_ERR_* code for
 * sizes the MoE entry points reject. A call of more tokens than one pass holds
 * (SMX_PLAN_CHUNK_TOKENS) runs its passes with the plan of their own sizes: this describes the
 * first. shared_I = 0: no shared expert.
 * No counterpart in the reference's operator API; it describes what replaces the reference's
 * per-call kernel configuration rule and grid (specmoe/layers/fused_moe_kernel.py:222-223,
 * 293-306), for tests and for the solver's performance model.
 */
enum smx_plan_field {
  SMX_PLAN_TILED = 0,           /* 1: tiled MFMA expert kernels; 0: weight-streaming kernels */
  SMX_PLAN_FUSED_DOWN,          /* 1: down projection fused with the combine (few tokens) */
  SMX_PLAN_SPAN,                /* sorted positions per work range */
  SMX_PLAN_MAX_RANGES,          /* work ranges the grids are sized for */
  SMX_PLAN_TOK_TILES,           /* 16-token tiles per range (streaming kernels) */
  SMX_PLAN_SPLITS,              /* K splits of the routed down projection */
  SMX_PLAN_SPLIT_STEPS,         /* 64-byte steps per down split */
  SMX_PLAN_DOWN_ROWS,           /* 16-row W2 tiles per down wave (streaming kernels) */
  SMX_PLAN_GATEUP_WAVES,        /* waves per gate/up workgroup (streaming kernels) */
  SMX_PLAN_GATEUP_KSPLIT,       /* 1: each gate/up item's K walk split between wave pairs */
  SMX_PLAN_SHARED_SPLITS,       /* K splits of the shared expert's down projection */
  SMX_PLAN_SHARED_SPLIT_STEPS,  /* 64-byte steps per shared down split */
  SMX_PLAN_SHARED_TOK_GROUPS,   /* token ranges of the shared expert */
  SMX_PLAN_SHARED_GATEUP_BLOCKS,/* leading gate/up workgroups running the shared expert */
  SMX_PLAN_SHARED_DOWN_BLOCKS,  /* leading down workgroups running the shared expert */
  SMX_PLAN_TILE_GATEUP_GRID,    /* tiled path: gate/up workgroups launched (0 otherwise) */
  SMX_PLAN_TILE_DOWN_GRID,      /* tiled path: down workgroups launched (0 otherwise) */
  SMX_PLAN_SINGLE_LAUNCH,       /* 1: one token in one launch (smx_set_single_launch_layer), when
                                   the routing runs inside it and the stream is not capturing */
  SMX_PLAN_SYNC_BLOCKS,         /* single launch: gate/up workgroups the down workgroups wait for */
  SMX_PLAN_SYNC_OFFSET,         /* single launch: workspace byte offset of their flags (8 bytes
                                   each), followed by the status word; -1 otherwise */
  SMX_PLAN_TOPK_IN_GATEUP,      /* 1: a call given router logits (in the activation dtype) runs
                                   the top-k inside the gate/up launch (no routing launch) */
  SMX_PLAN_EXPERT_ITEMS,        /* 1: a call whose gate/up launch routes the batch in its
                                   multi-wave form (given ids; given logits when
                                   SMX_PLAN_TOPK_IN_GATEUP is also 1) numbers its routed items
                                   by expert (smx_set_gateup_expert_items) */
  SMX_PLAN_CHUNK_TOKENS,        /* tokens per pass */
  SMX_PLAN_WORKSPACE_BYTES,     /* workspace of the whole call */
  SMX_PLAN_FIELDS
};
int smx_moe_plan_info(int64_t T, int64_t H, int64_t I, int64_t E, int64_t top_k,
                      int64_t shared_I, int dtype, int64_t* out, int n);

/*
 * Measurement hook. With `events` = 5 hipEvent_t handles, every following MoE call records
 * events[0] before routing and events[1..4] after the routing, gate/up, down and combine
 * kernels, on the call's stream; `events` = NULL (count 0) turns it off. Process-wide and
 * not thread-safe: for benchmarks only.
 * No counterpart in the reference's operator API; it plays the role of the reference's
 * CUDA-event timing around post_attention (specmoe/backend/execution_engine.py:450-451,
 * 740-741, 783-784), at kernel granularity.
 */
int smx_set_profile_events(void* const* events, int count);

/*
 * Measurement: reads `bytes` of device memory at `src` (16-byte aligned) in one launch, one
 * 256-thread workgroup per `bytes_per_workgroup` contiguous bytes (a multiple of 16 KiB that
 * divides `bytes`), with 16-byte non-temporal loads, four in flight per lane; `sink` (4 bytes of
 * device memory) is written only if the data's XOR equals a fixed marker. Timed around it, this
 * is the practical floor of a read of that size in one launch (launch, ramp and tail
 * included), which bench.py reports beside the expert kernels' small-batch launches.
 * No counterpart in the reference: measurement only.
 */
int smx_stream_read(const void* src, size_t bytes, size_t bytes_per_workgroup, void* sink,
                    void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SPECMOE_MI355X_H */
