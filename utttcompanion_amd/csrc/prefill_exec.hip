// One chunk of the chunk-first prefill with fast-weight writes, enqueued by one host call
// (reference uTTTModel's chunk-first forward, model/uttt_model.py:453-608: per chunk, every
// layer's block forward, model/uttt_layer.py:1528-1555, reading the chunk-start fast weights,
// then the layers' chained updates, :519-608).
//
// The work is the launches the per-call entry points make: per layer, the forward pass on the
// main stream, part 1 of chain stage l (the snapshot products with the chunk-start S and the
// key Gram rows, which need only the keys of layers <= l) after the layer's projections, and
// part 2 (the layer's update) after the layer's readout, both on the chain stream; then the
// state write after the last layer, which the main stream waits for.  (Part 1 on a third stream, beside part 2 of earlier layers,
// measured slower at config 3: 621 against 603 ms per prefill, the snapshot products then
// competing for HBM with the chain's streaming kernels and the readouts.)  The host side costs
// one call per chunk instead of one binding call per launch.
#include "uttt_host.h"

namespace uttt {
namespace {

int hip_status(hipError_t rc, const char* what) {
  return rc == hipSuccess ? UTTT_OK : fail(UTTT_ERR_HIP, "uttt_prefill_chunk: %s: %s", what, hipGetErrorString(rc));
}

}  // namespace
}  // namespace uttt

using namespace uttt;

#define UTTT_TRY(call)            \
  do {                            \
    const int rc_ = (call);       \
    if (rc_ != UTTT_OK) return rc_; \
  } while (0)

extern "C" int uttt_prefill_chunk(const uttt_prefill_chunk_args* a, uttt_stream_t main_stream,
                                  uttt_stream_t chain_stream) {
  UTTT_REQUIRE(a != nullptr && a->layers != nullptr && a->chain != nullptr, "args, layers and chain must be non-NULL");
  UTTT_REQUIRE(a->n_layers >= 1 && a->n_layers <= UTTT_MAX_CHAIN && a->n_layers == a->chain->layers,
               "n_layers (%d) must equal the chain's layer count (%lld), 1..%d", (int)a->n_layers,
               (long long)a->chain->layers, UTTT_MAX_CHAIN);
  UTTT_REQUIRE(a->start_pos >= 0 && a->kv_offset >= 0, "start_pos and kv_offset must be >= 0");
  UTTT_REQUIRE(main_stream != chain_stream, "the chain needs a stream of its own");
  UTTT_REQUIRE(a->defer_join == 0 || a->defer_join == 1, "defer_join must be 0 or 1");
  const int L = a->n_layers;
  UTTT_REQUIRE(a->events != nullptr && a->n_events >= 2 * L + 2,
               "events must hold 2 n_layers + 2 = %d caller-owned events, got %d", 2 * L + 2,
               a->events != nullptr ? (int)a->n_events : 0);
  for (int i = 0; i < 2 * L + 2; ++i) UTTT_REQUIRE(a->events[i] != nullptr, "events[%d] is NULL", i);
  hipStream_t ms = static_cast<hipStream_t>(main_stream), cs = static_cast<hipStream_t>(chain_stream);
  if (a->defer_join || a->wait_event != nullptr) {
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    UTTT_TRY(hip_status(hipStreamIsCapturing(ms, &status), "hipStreamIsCapturing"));
    UTTT_REQUIRE(status == hipStreamCaptureStatusNone,
                 "a deferred join (defer_join or wait_event) cannot be part of a graph capture: every captured "
                 "call joins its own state write");
  }
  hipEvent_t const* ev = reinterpret_cast<hipEvent_t const*>(a->events);

  uttt_chunk_chain_args chain = *a->chain;  // this chunk's mask and surprise row
  chain.token_mask = a->token_mask;
  chain.mask_row_stride = a->token_mask != nullptr ? a->mask_row_stride : 0;
  chain.surprise = a->surprise;
  hipEvent_t fwd_done = ev[2 * L], chain_done = ev[2 * L + 1];
  for (int l = 0; l < L; ++l) {
    const uttt_prefill_layer_calls& c = a->layers[l];
    uttt_rope_append_args rope = c.rope;
    rope.start_pos = a->start_pos;
    rope.kv_offset = a->kv_offset;
    uttt_swa_prefill_args attn = c.attn;
    attn.q_offset = a->kv_offset;
    attn.kv_len = a->kv_offset + attn.q_len;
    hipEvent_t projected = ev[2 * l], read = ev[2 * l + 1];
    // the QKV product in 128-row tiles without a k split (96 workgroups at config 3): alone on
    // the GPU the planner's 64-row tiles are faster (13.4 against 16.3 us), but here the product
    // shares the CUs with the chain stream, and the config-3 prefill measured 554 ms against 556
    // with a k split of 2 and 561-572 with the planner's tiles
    UTTT_TRY(linear_enqueue(&c.qkv, ms, 128));
    UTTT_TRY(uttt_rope_kv_append(&rope, ms));
    UTTT_TRY(uttt_swa_prefill(&attn, ms));
    UTTT_TRY(uttt_linear(&c.attn_out, ms));
    UTTT_TRY(uttt_linear(&c.proj, ms));
    UTTT_TRY(uttt_proj_epilogue(&c.epilogue, ms));
    UTTT_TRY(hip_status(hipEventRecord(projected, ms), "hipEventRecord"));
    if (l == 0 && a->wait_event != nullptr) {  // the previous chunk's state write, deferred to here
      UTTT_TRY(hip_status(hipStreamWaitEvent(ms, static_cast<hipEvent_t>(a->wait_event), 0), "hipStreamWaitEvent"));
    }
    UTTT_TRY(uttt_swiglu_readout(&c.readout, c.readout_workspace, c.readout_workspace_bytes, ms));
    UTTT_TRY(hip_status(hipEventRecord(read, ms), "hipEventRecord"));
    UTTT_TRY(uttt_linear(&c.uttt_out, ms));
    UTTT_TRY(hip_status(hipStreamWaitEvent(cs, projected, 0), "hipStreamWaitEvent"));
    UTTT_TRY(uttt_chunk_chain_stage_part(&chain, a->chain_workspace, a->chain_workspace_bytes, l, 1, cs));
    UTTT_TRY(hip_status(hipStreamWaitEvent(cs, read, 0), "hipStreamWaitEvent"));
    UTTT_TRY(uttt_chunk_chain_stage_part(&chain, a->chain_workspace, a->chain_workspace_bytes, l, 2, cs));
  }
  // the state write follows every reader of the chunk-start state; the next chunk's first
  // reader (layer 0's readout) follows it.  Without defer_join the chain stream's work ends in a
  // join back to the main stream here, which keeps the call capturable in a graph (a capture
  // must not end with a forked stream's work unjoined); with it, the caller hands the
  // state-write event to its next call
  UTTT_TRY(hip_status(hipEventRecord(fwd_done, ms), "hipEventRecord"));
  UTTT_TRY(hip_status(hipStreamWaitEvent(cs, fwd_done, 0), "hipStreamWaitEvent"));
  UTTT_TRY(uttt_chunk_chain_stage(&chain, a->chain_workspace, a->chain_workspace_bytes, L, cs));
  UTTT_TRY(hip_status(hipEventRecord(chain_done, cs), "hipEventRecord"));
  if (!a->defer_join) UTTT_TRY(hip_status(hipStreamWaitEvent(ms, chain_done, 0), "hipStreamWaitEvent"));
  return ok();
}

extern "C" int uttt_events_create(int32_t n, void** events) {
  UTTT_REQUIRE(events != nullptr && n >= 0, "events must be non-NULL and n >= 0");
  for (int32_t i = 0; i < n; ++i) events[i] = nullptr;
  for (int32_t i = 0; i < n; ++i) {
    hipEvent_t e = nullptr;
    const hipError_t rc = hipEventCreateWithFlags(&e, hipEventDisableTiming);
    if (rc != hipSuccess) {
      for (int32_t j = 0; j < i; ++j) (void)hipEventDestroy(static_cast<hipEvent_t>(events[j]));
      for (int32_t j = 0; j < i; ++j) events[j] = nullptr;
      return fail(UTTT_ERR_HIP, "uttt_events_create: %s", hipGetErrorString(rc));
    }
    events[i] = e;
  }
  return ok();
}

extern "C" int uttt_events_destroy(int32_t n, void* const* events) {
  UTTT_REQUIRE(events != nullptr && n >= 0, "events must be non-NULL and n >= 0");
  int status = UTTT_OK;
  for (int32_t i = 0; i < n; ++i) {
    if (events[i] == nullptr) continue;
    const hipError_t rc = hipEventDestroy(static_cast<hipEvent_t>(events[i]));
    if (rc != hipSuccess && status == UTTT_OK) status = fail(UTTT_ERR_HIP, "uttt_events_destroy: %s", hipGetErrorString(rc));
  }
  return status == UTTT_OK ? ok() : status;
}

extern "C" int uttt_stream_wait_event(uttt_stream_t stream, void* event) {
  UTTT_REQUIRE(event != nullptr, "event must be non-NULL");
  UTTT_TRY(hip_status(hipStreamWaitEvent(static_cast<hipStream_t>(stream), static_cast<hipEvent_t>(event), 0),
                      "hipStreamWaitEvent"));
  return ok();
}
