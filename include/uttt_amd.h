/*
 * uttt_amd.h -- C ABI of the MI355X (gfx950) uTTT hot-path library (libuttt_amd.so).
 *
 * Plain C: device pointers, int64 sizes/strides, scalars and a HIP stream.
 * Nothing here allocates or frees device memory and no call synchronises the
 * stream; every call only enqueues kernels on the stream it is given, so calls
 * are stream-ordered and safe to record into a HIP graph.  Buffers (including
 * workspace) belong to the caller; the one exception is the device-resident scratch
 * array of uttt_chunk_update_noalloc.  Every entry point returns UTTT_OK (0) or an
 * error code; uttt_last_error() then describes the failure (per host thread).
 *
 * Shapes follow the reference PyTorch modules of Phova/uTTTCompanion
 * (model/uttt_layer.py).  "Row" = one batch row / one request, each with its own
 * fp32 fast-weight state.  Layouts: activations (B, T, D) with the feature dim
 * contiguous and a token stride of D; state W_up/W_gate (B, D, F), W_down (B, F, D)
 * contiguous per row (row stride given separately; 0 = one matrix shared by all rows).
 */
#ifndef UTTT_AMD_H
#define UTTT_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* uttt_stream_t; /* a hipStream_t; NULL = the default stream */

enum { UTTT_DTYPE_F32 = 0, UTTT_DTYPE_BF16 = 1 };
enum { UTTT_OK = 0, UTTT_ERR_INVALID = 1, UTTT_ERR_HIP = 2, UTTT_ERR_WORKSPACE = 3 };

/* ABI version of the structures and entry points below: uttt_abi_version() returns it, and the
 * Python binding reads it from this header and refuses a library built from another one. */
#define UTTT_ABI_VERSION 24

/* Text of the last error on this host thread ("" when none). */
const char* uttt_last_error(void);
/* UTTT_ABI_VERSION of the header the library was built from. */
int uttt_abi_version(void);

/* ---------------------------------------------------------------------------
 * 1. Fused chunk fast-weight update + causal readout.
 *    Replaces fused_chunk_ttt_step (model/uttt_layer.py:414-534), i.e.
 *    analytical_swiglu_chunk_grad (:279-411) + clip (:468-489) + momentum and
 *    decay (:493-511) + inactive-row select (:513-520) + readout (:525-533),
 *    as called by SharedFastWeightPool.chunk_step (:697-771).
 * ------------------------------------------------------------------------- */
typedef struct {
  int64_t batch;      /* B rows */
  int64_t tokens;     /* C tokens in this chunk, 1..UTTT_MAX_UPDATE_TOKENS (one write for the whole
                         chunk; chunks longer than 64 run the 64-token kernels per block and a
                         separate pass for the chunk's clip norm) */
  int64_t d_model;    /* D, multiple of 64 */
  int64_t d_ff;       /* F, multiple of 64 */
  int32_t act_dtype;  /* UTTT_DTYPE_F32 or UTTT_DTYPE_BF16: q/k/v/eta/alpha/out */
  int32_t normalize_by_dim;
  float momentum_beta, max_inner_grad_norm, eps;
  /* chunk inputs, act_dtype; token stride D (eta/alpha: 1); row strides in elements */
  const void* q; int64_t q_row_stride;
  const void* k; int64_t k_row_stride;
  const void* v; int64_t v_row_stride;
  const void* eta; int64_t eta_row_stride;
  const void* alpha; int64_t alpha_row_stride;
  const float* token_mask; int64_t mask_row_stride; /* (B, C) fp32 or NULL */
  /* write cursor (fp32 master state), row stride = D*F */
  const float* w_up; const float* w_gate; const float* w_down;
  const float* s_up; const float* s_gate; const float* s_down;
  /* read snapshot for the readout (may equal the cursor); row stride 0 = shared */
  const float* r_up; const float* r_gate; const float* r_down; int64_t r_row_stride;
  const float* ln_weight; const float* ln_bias; /* (D,) fp32 */
  /* outputs: new state (may alias the cursor for in-place), readout, surprise */
  float* w_up_out; float* w_gate_out; float* w_down_out;
  float* s_up_out; float* s_gate_out; float* s_down_out;
  void* out; int64_t out_row_stride; /* (B, C, D) act_dtype */
  float* surprise;                   /* device scalar (fp32): batch-global mean token loss (L:369-380) */
  float* row_loss;                   /* optional (B, 2) fp32: per row [sum of masked token losses,
                                        valid tokens], for per-request surprise; NULL to skip */
  float min_row_surprise;            /* > 0: a row whose masked mean token loss in this chunk is
                                        below it keeps W and S (per-chunk surprise gate; not in the
                                        reference, whose gate is per turn, P:524-551); 0 = off */
} uttt_chunk_update_args;

size_t uttt_chunk_update_workspace(int64_t batch, int64_t d_model, int64_t d_ff, int32_t act_dtype);
/* The same for chunks of up to `tokens` tokens (the reference's configs write 128- and 512-token
 * chunks: configs/5090_config.yaml:31, configs/5090_pretrain_20261029.yaml:28); 0 if invalid. */
#define UTTT_MAX_UPDATE_TOKENS 512
size_t uttt_chunk_update_workspace_tokens(int64_t batch, int64_t tokens, int64_t d_model, int64_t d_ff,
                                          int32_t act_dtype);
int uttt_chunk_update(const uttt_chunk_update_args* args, void* workspace, size_t workspace_bytes,
                      uttt_stream_t stream);

/* The same update as UTTT_UPDATE_PHASES stream-ordered launches, one per call, in order
 * 0..4 on one stream with one workspace: 0 U/G/H (both paths), 1 Z partial sums,
 * 2 LayerNorm + loss + dZ + readout, 3 dH/dU/dG + gradient-norm partials (for a chunk of more
 * than 64 tokens, a second launch forms them from every token block), 4 clip/momentum/
 * decay/select applied to W and S.  Running all five equals uttt_chunk_update; it exists
 * so a caller can place timing events (or other stream work) between the phases. */
#define UTTT_UPDATE_PHASES 5
int uttt_chunk_update_phase(const uttt_chunk_update_args* args, void* workspace, size_t workspace_bytes,
                            int32_t phase, uttt_stream_t stream);

/* The same update with no workspace argument and no device allocation.  It has no counterpart in
 * the reference: it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The workspace is a
 * device-resident array of UTTT_NOALLOC_SCRATCH_BYTES inside the library (each GPU the library
 * runs on holds its own copy until the process ends); shapes whose workspace
 * (uttt_chunk_update_workspace_tokens) exceeds it are refused with UTTT_ERR_INVALID.  The stream's device
 * must be the current device.  Every call on one GPU uses that GPU's array, so calls that overlap
 * on one GPU (other streams, other host threads) race: order them.  Results equal
 * uttt_chunk_update's. */
#define UTTT_NOALLOC_SCRATCH_BYTES (64ull << 20)
int uttt_chunk_update_noalloc(const uttt_chunk_update_args* args, uttt_stream_t stream);

/* ---------------------------------------------------------------------------
 * 1a. Every chunk of one standalone layer's forward in one call.
 *     Replaces the per-chunk chunk_step loop of uTTTLayer.forward
 *     (model/uttt_layer.py:1451-1478) for one row of fp32 activations: chunk c
 *     (tokens [c * chunk_size, min(T, (c + 1) * chunk_size))) is the update of
 *     uttt_chunk_update applied to the state left by chunk c - 1, with the readout
 *     through that chunk's pre-update state (read_state None).  The updates run in
 *     persistent launches of up to 16 chunks: each workgroup keeps 8 columns of
 *     W_up / W_gate and rows of W_down and their momentum on chip from the first
 *     chunk of a launch to the last, and the workgroups meet at three device-wide
 *     barriers per chunk, so a launch needs d_ff / 8 workgroups resident at once
 *     (at most one per CU).  Each launch saves its chunks' query H and W_down for
 *     the readout, which follows it on the stream.
 *     q/k/v/out (T, D) row-major; eta/alpha/token_mask (T,); surprise (n_chunks,)
 *     receives each chunk's surprise.  The state outputs may alias the inputs.
 *     A barrier that waits past its bound (about a second) sets the flag word at
 *     uttt_layer_update_resident_flag_offset in the workspace (cleared by every call)
 *     and no later barrier waits, so every workgroup still runs to its end; the call's
 *     results are then invalid, and it writes NaN into its output state, surprise and
 *     (for the chunks from the failing launch on) readout.
 * ------------------------------------------------------------------------- */
typedef struct {
  int64_t batch;       /* must be 1 */
  int64_t tokens;      /* T >= 1 */
  int64_t d_model;     /* 128, 256 or 512 */
  int64_t d_ff;        /* a multiple of 64, d_ff / 8 <= the device's CUs */
  int64_t chunk_size;  /* 1..64 */
  int32_t normalize_by_dim;
  float momentum_beta, max_inner_grad_norm, eps;
  const float* q; const float* k; const float* v;
  const float* eta; const float* alpha; const float* token_mask; /* token_mask NULL = all valid */
  const float* w_up; const float* w_gate; const float* w_down;
  const float* s_up; const float* s_gate; const float* s_down;
  const float* ln_weight; const float* ln_bias;
  float* w_up_out; float* w_gate_out; float* w_down_out;
  float* s_up_out; float* s_gate_out; float* s_down_out;
  float* out;
  float* surprise;
  unsigned* error_word;  /* optional device word (NULL = none): set to 1 when a barrier timed out;
                            never cleared by the library, so it collects the failures of many calls */
  int32_t force_timeout; /* test hook, normally 0: nonzero runs the call as if its first barrier had
                            timed out (flag and error word set before the first launch, no barrier
                            waits, every kernel runs to its end, NaN results) */
} uttt_layer_update_args;

int uttt_layer_update_resident_supported(int64_t batch, int64_t d_model, int64_t d_ff);
size_t uttt_layer_update_resident_workspace(int64_t d_model, int64_t d_ff);
size_t uttt_layer_update_resident_flag_offset(int64_t d_model, int64_t d_ff);
int uttt_layer_update_resident(const uttt_layer_update_args* args, void* workspace, size_t workspace_bytes,
                               uttt_stream_t stream);

/* ---------------------------------------------------------------------------
 * 1b. One chunk's updates for all L layers of the chunk-first shared schedule.
 *     Replaces the per-layer chunk_step calls that uTTTModel._run_shared_chunk /
 *     _run_shared_layer_segment (model/uttt_model.py:519-608) make for one chunk: layer l's
 *     update (model/uttt_layer.py:414-534, loss / clip / momentum / decay / inactive rows as
 *     in uttt_chunk_update) is applied to the state left by layers 0..l-1, starting from the
 *     chunk-start state.  Every layer's readout reads the chunk-start state, so readouts are
 *     not part of this call (uttt_swiglu_readout over that state or its bf16 copies).
 *     The state is updated in place, once.  Layer l's inputs are given per layer:
 *     k/v (batch, tokens, d_model) with token stride d_model and row stride kv_row_stride,
 *     eta/alpha (batch, tokens) with token stride 1 and row stride ea_row_stride.
 * ------------------------------------------------------------------------- */
#define UTTT_MAX_CHAIN 64
typedef struct {
  int64_t batch, layers, tokens, d_model, d_ff; /* layers <= UTTT_MAX_CHAIN, tokens <= 64 */
  int32_t act_dtype, normalize_by_dim;
  float momentum_beta, max_inner_grad_norm, eps;
  float min_row_surprise;            /* > 0: per-chunk surprise gate per layer (not in the reference) */
  const void* k[UTTT_MAX_CHAIN];
  const void* v[UTTT_MAX_CHAIN];
  int64_t kv_row_stride;
  const void* eta[UTTT_MAX_CHAIN];
  const void* alpha[UTTT_MAX_CHAIN];
  int64_t ea_row_stride;
  const float* token_mask; int64_t mask_row_stride; /* optional (batch, >= tokens) fp32, all layers */
  float* w_up; float* w_gate; float* w_down;        /* fp32 (B, D, F), (B, D, F), (B, F, D); in/out */
  float* s_up; float* s_gate; float* s_down;
  const float* ln_weight; const float* ln_bias;     /* (D,) fp32 */
  /* optional bf16 copies of the state (bf16 activations only, all six or none): on entry they
     hold the chunk-start state rounded to bf16 and are what the kernels read in place of the
     fp32 masters (the reference rounds W to the activation dtype for these products); on exit
     they hold the final state rounded to bf16 */
  void* w_up_copy; void* w_gate_copy; void* w_down_copy;
  void* s_up_copy; void* s_gate_copy; void* s_down_copy;
  float* surprise;                   /* (layers,) batch-global surprise of each layer */
  float* row_loss;                   /* optional (layers, batch, 2): [sum of masked token losses, valid tokens] */
  /* nonzero (bf16 copies only): layer l's products k_l W_up and k_l W_gate with the chunk-start
   * state are written by the caller into the workspace slots uttt_chunk_chain_w_products names
   * (uttt_swiglu_readout with keys) before stage l's second part runs; the stages form only the
   * S products */
  int32_t w_products_given;
} uttt_chunk_chain_args;

size_t uttt_chunk_chain_workspace(int64_t batch, int64_t layers, int64_t d_model, int64_t d_ff, int32_t act_dtype);
int uttt_chunk_chain(const uttt_chunk_chain_args* args, void* workspace, size_t workspace_bytes,
                     uttt_stream_t stream);
/* The same chain as layers + 1 stream-ordered stages, one per call, in order on one stream
 * with one workspace.  Layers run in groups: one layer each while 8 * d_model * d_ff * batch
 * bytes (the state read of one group's products) is at most 128 MiB, else groups of 4 with the
 * last layer alone.  The stage of a group's last layer forms the group's products with the
 * chunk-start state and its key Gram rows, and runs each of its layers (forward / backward
 * through the state left by the layers before it, the previous layer's clip / decay step);
 * the other stages of a group launch nothing.  Stage `layers` is the last layer's step and
 * the state write.
 * Stage l reads only layers <= l, so only their k/v/eta/alpha pointers need to be set: a
 * caller can run stage l (on a second stream) as soon as layer l's inputs exist, while it
 * computes the next layers' forward passes.  The state write must follow every reader of the
 * chunk-start state (the readouts).  Running every stage equals uttt_chunk_chain. */
int uttt_chunk_chain_stage(const uttt_chunk_chain_args* args, void* workspace, size_t workspace_bytes,
                           int32_t stage, uttt_stream_t stream);
/* One part of stage `stage`: part 1 launches its snapshot products and key Gram rows (they read
 * only the keys of layers <= stage and the chunk-start state), part 2 the rest; part 1 then part
 * 2 on one stream equals uttt_chunk_chain_stage (part 0).  Part 1 of stage l may run beside
 * part 2 of any stage m < l (on another stream, the parts 1 in order on theirs): they touch
 * disjoint workspace slots.  With
 * w_products_given, part 2 of stage l must follow the caller's writes of layer l's products. */
int uttt_chunk_chain_stage_part(const uttt_chunk_chain_args* args, void* workspace, size_t workspace_bytes,
                                int32_t stage, int32_t part, uttt_stream_t stream);
/* Some of the launches of a stage part (part 0: the whole stage), e.g. to time single kernels with
 * events between them: the launches a part makes are numbered 0, 1, ... in enqueue order, and the
 * call enqueues those numbered in [launch_begin, launch_end) (none when launch_end <=
 * launch_begin); enqueueing consecutive ranges in order on one stream equals
 * uttt_chunk_chain_stage_part.  *count (if not NULL) receives the number of launches of the part
 * and names[i] (i < names_cap) the kernel name of launch i (static strings).  A range past the
 * count is an error. */
int uttt_chunk_chain_stage_launch(const uttt_chunk_chain_args* args, void* workspace, size_t workspace_bytes,
                                  int32_t stage, int32_t part, int32_t launch_begin, int32_t launch_end,
                                  const char** names, int32_t names_cap, int32_t* count, uttt_stream_t stream);
/* Byte offsets in the chain workspace of layer `layer`'s k W_up and k W_gate products
 * ((batch, 64, d_ff) in the activation dtype, row stride 64 * d_ff). */
int uttt_chunk_chain_w_products(int64_t batch, int64_t layers, int64_t d_model, int64_t d_ff, int32_t act_dtype,
                                int32_t layer, size_t* up_offset, size_t* gate_offset);

/* ---------------------------------------------------------------------------
 * 1c. Slow-projection epilogue.  Replaces the RMSNorm / sigmoid part of
 *     fused_slow_projections (model/uttt_layer.py:1193-1231): from the packed product
 *     y = x [W_q; W_k; W_v; w_eta; w_alpha]^T + bias, one row (3 d_model + 2 values) per token,
 *     q = RMSNorm(y_q) * q_weight, k = RMSNorm(y_k) * k_weight, v = RMSNorm(y_v),
 *     eta = inner_lr * sigmoid(y_eta), alpha = weight_decay * sigmoid(y_alpha).
 *     q, k, v rows share out_row_stride; eta and alpha are contiguous (rows,).
 * ------------------------------------------------------------------------- */
typedef struct {
  int64_t rows, d_model;             /* d_model <= 4096 */
  int32_t act_dtype;
  float eps, inner_lr, weight_decay;
  const void* y; int64_t y_row_stride;
  const void* q_weight; const void* k_weight; /* (d_model,) in the activation dtype */
  void* q; void* k; void* v; int64_t out_row_stride;
  void* eta; void* alpha;
  /* Optional RMSNorm of the projection input folded into this step (NULL x: none): y was
   * projected from the un-normalised rows x (row stride x_row_stride, d_model wide) with the
   * norm weight folded into the projection weight and without bias; row r of y is scaled by
   * 1 / sqrt(mean(x_r^2) + x_eps), and the eta / alpha biases (2 values, activation dtype) are
   * added to its last two entries, before the epilogue proper. */
  const void* x; int64_t x_row_stride; float x_eps;
  const void* eta_alpha_bias;
} uttt_proj_epilogue_args;

int uttt_proj_epilogue(const uttt_proj_epilogue_args* args, uttt_stream_t stream);

/* ---------------------------------------------------------------------------
 * 2. Frozen fast-weight readout f_W(x) = x + LN((SiLU(x W_gate) * x W_up) W_down).
 *    Replaces swiglu_fast_forward (model/uttt_layer.py:211-247) as used by
 *    SharedFastWeightPool.forward_readout (:670-695) and the packed inference
 *    readout swiglu_packed_forward (:250-257) / CUDAGraphDecoder (engine/inference.py:263-276).
 * ------------------------------------------------------------------------- */
typedef struct {
  int64_t batch, tokens, d_model, d_ff; /* tokens: any T >= 1 */
  int32_t act_dtype;
  int32_t w_dtype;   /* UTTT_DTYPE_F32 masters, or UTTT_DTYPE_BF16 read copies (bf16 activations only) */
  float eps;
  const void* x; int64_t x_row_stride;
  const void* w_up; const void* w_gate; const void* w_down; int64_t w_row_stride; /* 0 = shared */
  const float* ln_weight; const float* ln_bias;
  void* out; int64_t out_row_stride;
  /* Optional key products for the layer chain (NULL keys: none; bf16 activations, tokens <= 64):
   * keys (batch, tokens, d_model), token stride d_model, row stride keys_row_stride; the call
   * also writes keys W_up and keys W_gate (batch, 64, d_ff) in the activation dtype at
   * key_up_out / key_gate_out (rows past tokens are 0), from the same weight reads as the readout,
   * equal to the products uttt_chunk_chain forms itself (no counterpart in the reference: the
   * snapshot products of SharedFastWeightPool.update_fast_weights' dual form, shared with the
   * readout's reads of the same chunk-start weights). */
  const void* keys; int64_t keys_row_stride;
  void* key_up_out; void* key_gate_out;
  /* Optional, one bf16 token per row (tokens == 1, no keys, d_model <= 2048):
   * x_norm_weight (d_model, activation dtype) reads out RMSNorm(x) with that weight and eps
   * x_norm_eps instead of x, rounded to the activation dtype as the separate norm rounds it (the
   * residual term is the normalised row too): the decode step's q_norm before the readout
   * (reference uTTTLayer's rms_norm of the query projection, model/uttt_layer.py:1528-1555).
   * row_counters (batch uint32, zero before the first call; every call leaves them zero) lets the
   * LayerNorm and residual run in each row's last weight block, so the call is one launch;
   * calls that share counters must not overlap.  NULL: a second launch does the LayerNorm. */
  const void* x_norm_weight; float x_norm_eps;
  uint32_t* row_counters;
  /* One bf16 token per row only (ignored otherwise): nonzero walks every row's weight blocks in
   * descending order.  The decode step's readouts of consecutive layers read the same
   * per-request copies; alternating the direction lets each call start on the lines the previous
   * call read last, which the 256 MB infinity cache still holds (measured at 32 requests,
   * d_model 768, d_ff 2048: 1.08 against 1.12 ms per 12-layer decode step).  The result differs
   * from the ascending walk only by the order of the fp32 sums. */
  int32_t sweep_reverse;
} uttt_readout_args;

size_t uttt_readout_workspace(int64_t batch, int64_t tokens, int64_t d_model, int64_t d_ff, int32_t act_dtype);
int uttt_swiglu_readout(const uttt_readout_args* args, void* workspace, size_t workspace_bytes,
                        uttt_stream_t stream);

/* ---------------------------------------------------------------------------
 * 3. RoPE on q/k + KV append.  Replaces RotaryEmbedding.forward + apply_rope
 *    (model/uttt_layer.py:935-958) and the cache concatenation (:1082-1102).
 *    q is rotated in place; rotated k and v are written into the caller's KV
 *    buffers at time index kv_offset + t.  Position of token t = start_pos + t.
 *    cos/sin: fp32 tables (positions, head_dim) built as in RotaryEmbedding._build_cache (:910-933).
 * ------------------------------------------------------------------------- */
typedef struct {
  int64_t batch, tokens, n_heads, n_kv_heads, head_dim;
  int32_t act_dtype;
  int64_t start_pos, table_len;
  const float* cos_table; const float* sin_table;
  void* q; int64_t q_stride_b, q_stride_t, q_stride_h;       /* rotated in place */
  const void* k; int64_t k_stride_b, k_stride_t, k_stride_h;
  const void* v; int64_t v_stride_b, v_stride_t, v_stride_h;
  void* k_cache; void* v_cache; int64_t kv_stride_b, kv_stride_h, kv_stride_t; int64_t kv_offset;
  /* Optional RMSNorm of the projection input folded into this step (NULL x: none).  q / k / v
   * were projected from the un-normalised rows x with the norm weight folded into the
   * projection weight; token t's q / k / v are scaled by 1 / sqrt(mean(x_t^2) + x_eps) first. */
  const void* x; int64_t x_stride_b, x_stride_t, x_dim; float x_eps;
} uttt_rope_append_args;

int uttt_rope_kv_append(const uttt_rope_append_args* args, uttt_stream_t stream);

/* ---------------------------------------------------------------------------
 * 4. Sliding-window GQA attention for prefill / multi-token steps.
 *    Replaces the SDPA / FlexAttention dispatch of SlidingWindowAttention.forward
 *    (model/uttt_layer.py:1119-1165) with its mask (:1028-1056): query i (absolute
 *    key index q_offset + i) sees key j iff 0 <= q_offset + i - j < window and
 *    j < kv_len; kv head = h / (n_heads / n_kv_heads); softmax scale 1/sqrt(head_dim).
 * ------------------------------------------------------------------------- */
typedef struct {
  int64_t batch, n_heads, n_kv_heads, q_len, kv_len, head_dim; /* head_dim 64 or 128 */
  int64_t q_offset, window;
  int32_t act_dtype; /* bf16 or fp32 */
  float scale;
  const void* q; int64_t q_stride_b, q_stride_h, q_stride_t;
  const void* k; int64_t k_stride_b, k_stride_h, k_stride_t;
  const void* v; int64_t v_stride_b, v_stride_h, v_stride_t;
  void* out; int64_t o_stride_b, o_stride_h, o_stride_t;
  void* workspace; size_t workspace_bytes; /* >= uttt_swa_prefill_workspace(...) */
} uttt_swa_prefill_args;

size_t uttt_swa_prefill_workspace(int64_t batch, int64_t n_heads, int64_t q_len, int64_t kv_len, int64_t head_dim,
                                  int64_t window);
int uttt_swa_prefill(const uttt_swa_prefill_args* args, uttt_stream_t stream);

/* ---------------------------------------------------------------------------
 * 5. One decode step over ring-buffer SWA KV caches for N independent requests.
 *    Replaces CUDAGraphDecoder._forward's per-layer ring write + masked SDPA
 *    (engine/inference.py:244-259) and the eager seq_len==1 branch
 *    (model/uttt_layer.py:1082-1124).  Request n at position p = positions[n]:
 *    RoPE at p (when tables are given), k/v written to slot p mod window, then
 *    attention over slots < min(p + 1, window).
 * ------------------------------------------------------------------------- */
typedef struct {
  int64_t n_req, n_heads, n_kv_heads, head_dim, window;
  int32_t act_dtype;
  float scale;
  const int64_t* positions;                      /* device, (N,) */
  const float* cos_table; const float* sin_table; int64_t table_len; /* NULL: inputs pre-rotated */
  const void* q; int64_t q_stride_n;             /* (N, H, hd), head stride hd */
  const void* k_new; const void* v_new; int64_t kv_new_stride_n; /* (N, Hkv, hd) */
  void* k_ring; void* v_ring; int64_t ring_stride_n; /* (N, Hkv, window, hd) */
  void* out; int64_t o_stride_n;                 /* (N, H, hd) */
  void* workspace; size_t workspace_bytes;       /* >= uttt_swa_decode_workspace(...): the split
                                                    partials of the general form (calls sharing it
                                                    must be ordered) */
} uttt_swa_decode_args;

size_t uttt_swa_decode_workspace(int64_t n_req, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                                 int64_t window);
int uttt_swa_decode(const uttt_swa_decode_args* args, uttt_stream_t stream);

/* ---------------------------------------------------------------------------
 * 6. Slow-anchor elastic pull W <- (1 - lambda) W + lambda W_0 with an optional
 *    per-row drift ceiling |W - W_0| <= ratio |W_0|.  Replaces
 *    SharedFastWeightPool.apply_elastic_pull (model/uttt_layer.py:773-832).
 *    ratio <= 0 disables the ceiling.  out_* may alias w_* (in place).
 * ------------------------------------------------------------------------- */
typedef struct {
  int64_t batch, d_model, d_ff;
  float anchor_lambda, max_drift_ratio;
  const float* w_up; const float* w_gate; const float* w_down;    /* (B, D, F), (B, D, F), (B, F, D) */
  const float* w0_up; const float* w0_gate; const float* w0_down; /* (D, F), (D, F), (F, D) */
  float* out_up; float* out_gate; float* out_down;
} uttt_elastic_pull_args;

size_t uttt_elastic_pull_workspace(int64_t batch);
int uttt_elastic_pull(const uttt_elastic_pull_args* args, void* workspace, size_t workspace_bytes,
                      uttt_stream_t stream);

/* 7. Squared drift norms for SharedFastWeightPool.compute_drift (model/uttt_layer.py:834-874):
 *    out6[0..2] = sum over rows of |W_m - W0_m|^2 (up, gate, down), out6[3..5] = |W0_m|^2.
 *    Uses the elastic-pull workspace size. */
int uttt_fast_weight_drift(int64_t batch, int64_t d_model, int64_t d_ff,
                           const float* w_up, const float* w_gate, const float* w_down,
                           const float* w0_up, const float* w0_gate, const float* w0_down,
                           float* out6, void* workspace, size_t workspace_bytes, uttt_stream_t stream);

/* ---------------------------------------------------------------------------
 * 8. Skinny slow-weight product out = x W^T (+ residual) for a few rows, bf16 operands with
 *    fp32 accumulation.  Replaces the F.linear calls of the batched decode step
 *    (engine/inference.py:263-276: the packed q/k/v projection, the uTTT query projection),
 *    the residual projections h + linear(x) (model/uttt_layer.py:1528-1555) and the LM head
 *    when one token per request is stepped.  x (m, k), w (n, k) row-major, out (m, n);
 *    residual (m, n) may be NULL or alias out.  m <= 64, n % 32 == 0, k % 64 == 0.
 *    x_eps > 0 folds an input RMSNorm in (the block's attn_norm / uttt_norm, the final norm
 *    before the LM head): each row of x is scaled by 1 / sqrt(mean(x^2) + x_eps) and w must
 *    carry the norm weight multiplied into its columns.  x_eps = 0: plain product.
 * ------------------------------------------------------------------------- */
typedef struct {
  int64_t m, n, k;
  int32_t act_dtype; /* UTTT_DTYPE_BF16 */
  float x_eps;
  const void* x; int64_t x_row_stride;
  const void* w; int64_t w_row_stride;
  const void* residual; int64_t residual_row_stride;
  void* out; int64_t out_row_stride;
} uttt_skinny_linear_args;

int uttt_skinny_linear(const uttt_skinny_linear_args* args, uttt_stream_t stream);

/* ---------------------------------------------------------------------------
 * 8b. Slow-weight product out = x W^T (+ residual) for many rows, bf16 operands with fp32
 *     accumulation.  Replaces the F.linear / h + linear(x) calls of the chunk-first forward pass
 *     (model/uttt_layer.py:1058-1081 the packed QKV projection, :1193-1231 the packed uTTT
 *     projections, :1528-1555 the block residual projections) at m = rows x chunk tokens.
 *     x (m, k), w (n, k) row-major with row strides >= k (multiples of 8 elements, 16-byte
 *     aligned bases), out (m, n); residual (m, n) may be NULL or alias out.  k % 64 == 0.
 *     Calls that share a workspace must not overlap.
 * ------------------------------------------------------------------------- */
typedef struct {
  int64_t m, n, k;
  int32_t act_dtype; /* UTTT_DTYPE_BF16 */
  const void* x; int64_t x_row_stride;
  const void* w; int64_t w_row_stride;
  const void* residual; int64_t residual_row_stride;
  void* out; int64_t out_row_stride;
  void* workspace; size_t workspace_bytes; /* zero-filled once; left zero-filled by every call */
} uttt_linear_args;

/* Workspace bytes uttt_linear needs for this shape on the current device (0: none; the k loop
 * is split over several workgroups per output tile only when the tiles do not cover the GPU). */
size_t uttt_linear_workspace(int64_t m, int64_t n, int64_t k);
int uttt_linear(const uttt_linear_args* args, uttt_stream_t stream);

/* ---------------------------------------------------------------------------
 * 8c. One chunk of the chunk-first prefill with fast-weight writes in one call.  Replaces the
 *     per-chunk loop body of uTTTModel's chunk-first forward (model/uttt_model.py:453-608: per
 *     layer the block forward of model/uttt_layer.py:1528-1555 through the chunk-start fast
 *     weights, then the chained updates of :519-608).  Per layer l, on main_stream: the packed
 *     QKV product (attention input norm folded), RoPE + KV append, sliding-window attention,
 *     the attention output product into the residual rows, the packed uTTT projection product
 *     and its epilogue, the readout (with the chain's key products) and the uTTT output product
 *     into the residual rows; on chain_stream: part 1 of chain stage l after layer l's
 *     epilogue, part 2 after its readout.  Then the state write (stage n_layers) on
 *     chain_stream after every layer, and main_stream waits for it.  Each layer's calls are
 *     the argument structs of the entry points above, built once for a prefill; the executor
 *     sets the per-chunk fields (rope start_pos / kv_offset, attention q_offset / kv_len =
 *     kv_offset + q_len, the chain's token_mask / mask_row_stride / surprise) in its own copies.
 *     The chain args must already name every layer's k / v / eta / alpha (the epilogue's
 *     outputs).  The call keeps no state between calls: the events that order the two streams
 *     belong to the caller (created with uttt_events_create), and a deferred join is handed to
 *     the next call explicitly (defer_join, wait_event).  Concurrent calls from several host
 *     threads must use distinct event sets.  A failing call may leave part of the chunk enqueued.
 * ------------------------------------------------------------------------- */
typedef struct {
  uttt_linear_args qkv;
  uttt_rope_append_args rope;
  uttt_swa_prefill_args attn;
  uttt_linear_args attn_out;
  uttt_linear_args proj;
  uttt_proj_epilogue_args epilogue;
  uttt_readout_args readout;
  void* readout_workspace; size_t readout_workspace_bytes;
  uttt_linear_args uttt_out;
} uttt_prefill_layer_calls;

typedef struct {
  int32_t n_layers;                        /* == chain->layers */
  const uttt_prefill_layer_calls* layers;  /* n_layers entries */
  const uttt_chunk_chain_args* chain;
  void* chain_workspace; size_t chain_workspace_bytes;
  int64_t start_pos;                       /* RoPE position of the chunk's first token */
  int64_t kv_offset;                       /* KV index of the chunk's first token */
  const float* token_mask; int64_t mask_row_stride; /* (batch, >= tokens) fp32 or NULL */
  float* surprise;                         /* (n_layers,) */
  /* nonzero: main_stream does not wait for this chunk's state write (recorded into
   * events[2 n_layers + 1]); the caller passes that event as the next call's wait_event, whose
   * main_stream waits for it just before layer 0's readout (the state's first reader), so that
   * call's layer-0 QKV .. epilogue overlap the state write.  The state write reads layer 0's
   * k / v / eta / alpha: the next call's layer-0 epilogue must write other buffers (the caller
   * alternates two sets).  The last call of a sequence passes 0.  Refused (UTTT_ERR_INVALID,
   * nothing enqueued) while main_stream is capturing: a capture must not end with the chain
   * stream unjoined. */
  int32_t defer_join;
  /* caller-owned hipEvent_t handles (uttt_events_create), n_events >= 2 n_layers + 2: two per
   * layer (projections done, readout done), then the forward's end and the state write */
  void* const* events; int32_t n_events;
  /* NULL, or the state-write event of a previous call made with defer_join: main_stream waits
   * for it before layer 0's readout.  Refused while main_stream is capturing (the event was
   * recorded outside the capture). */
  void* wait_event;
} uttt_prefill_chunk_args;

int uttt_prefill_chunk(const uttt_prefill_chunk_args* args, uttt_stream_t main_stream, uttt_stream_t chain_stream);

/* Event plumbing for uttt_prefill_chunk (no counterpart in the reference: its chunk-first
 * prefill, model/uttt_model.py:453-608, runs on one stream): n events created on the current
 * device with timing disabled, destroyed, and a stream made to wait for one (the join a caller
 * owes the main stream after a deferred call it does not follow up, e.g. on an exception). */
int uttt_events_create(int32_t n, void** events);
int uttt_events_destroy(int32_t n, void* const* events);
int uttt_stream_wait_event(uttt_stream_t stream, void* event);

/* ---------------------------------------------------------------------------
 * 9. Greedy next-token selection: per row, argmax of the logits with the excluded ids and the
 *    ids >= active_limit set to -inf first (torch.argmax semantics: NaN is the largest value,
 *    ties go to the lowest id).  Replaces the temperature-0 branch of
 *    uTTTModel.sample_next_token (model/uttt_model.py:1203-1221) as the decode step uses it.
 *    active_limit < 0 or >= vocab: no limit.
 * ------------------------------------------------------------------------- */
typedef struct {
  int64_t rows, vocab;
  int32_t dtype;    /* UTTT_DTYPE_BF16 or UTTT_DTYPE_F32 logits */
  int32_t n_banned; /* <= 8 */
  int32_t banned[8];
  int64_t active_limit;
  const void* logits; int64_t row_stride;
  int64_t* out;     /* (rows,) token ids */
  int64_t* advance; /* optional (rows,): each entry is incremented by one (a decode step's position
                     * counters, advanced in the same launch); NULL: none */
} uttt_greedy_args;

int uttt_greedy_select(const uttt_greedy_args* args, uttt_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* UTTT_AMD_H */
