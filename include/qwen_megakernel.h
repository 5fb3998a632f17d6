/*
 * C ABI of the MI355X (gfx950) Qwen3 decode library, libqwen_megakernel_amd.so.
 *
 * Plain pointers, sizes and a HIP stream; no torch types.  The first three
 * entry points are the reference's launchers with the same names, argument
 * order and meaning, with hipStream_t in place of cudaStream_t:
 *
 *   launch_ldg_decode_direct      <- reference csrc/kernel.cu:1477-1505
 *                                    (declared csrc/torch_bindings.cpp:45-53)
 *   launch_ldg_decode_persistent  <- reference csrc/kernel.cu:1507-1543
 *                                    (declared csrc/torch_bindings.cpp:35-43)
 *   launch_ldg_generate_nosync    <- reference csrc/kernel.cu:1547-1605
 *                                    (declared csrc/torch_bindings.cpp:83-91)
 *
 * All tensors are device pointers.  Layout (as in the reference):
 *   embed_weight / lm_head_weight  bf16 [vocab][hidden] (tied in Qwen3-0.6B)
 *   layer_weights                  device array of num_layers LDGLayerWeights
 *   cos_table / sin_table          bf16 [max_seq_len][head_dim]
 *   k_cache / v_cache              bf16 [num_layers][num_kv_heads][max_seq_len][head_dim]
 *                                  (need not be zeroed: rows at or past a step's
 *                                  position never reach its output, NaN included)
 *   hidden_buffer                 bf16 [hidden]   receives the final hidden state
 *   g_normalized                   f32  [hidden]   receives the final-norm output
 * The other scratch pointers of the reference signature (g_activations,
 * g_residual, g_q, g_k, g_v, g_attn_out, g_mlp_intermediate, block_max_vals,
 * block_max_idxs) are accepted and not used: activations move between
 * workgroups through the library's own per-stream exchange buffers.
 *
 * Errors: the reference reports none.  Here every entry point validates its
 * arguments before launching (nothing is launched on error), and records a
 * status readable with qmk_last_status() on the calling thread.  Errors
 * found on the device (bounded waits that expired, a position outside the
 * cache in persistent mode) are latched per stream: later launches on that
 * stream do nothing until qmk_reset(); qmk_device_error() reports them.
 */
#ifndef QWEN_MEGAKERNEL_AMD_H
#define QWEN_MEGAKERNEL_AMD_H

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Per-layer weight table, same field order as the reference's
 * LDGLayerWeights (csrc/torch_bindings.cpp:21-33, csrc/kernel.cu:76-88). */
typedef struct LDGLayerWeights {
  const void *input_layernorm_weight;
  const void *q_proj_weight;
  const void *k_proj_weight;
  const void *v_proj_weight;
  const void *q_norm_weight;
  const void *k_norm_weight;
  const void *o_proj_weight;
  const void *post_attn_layernorm_weight;
  const void *gate_proj_weight;
  const void *up_proj_weight;
  const void *down_proj_weight;
} LDGLayerWeights;

/* Status codes (qmk_last_status). */
enum {
  QMK_OK = 0,
  QMK_ERR_ARG = 1,        /* invalid argument (null pointer, range) */
  QMK_ERR_POSITION = 2,   /* position outside [0, max_seq_len) */
  QMK_ERR_DEVICE = 3,     /* device unsuitable (needs 256 CUs, gfx950) */
  QMK_ERR_HIP = 4,        /* a HIP runtime call failed */
  QMK_ERR_POISONED = 5,   /* a previous launch on this stream failed; call qmk_reset */
  QMK_ERR_INIT = 6,       /* qmk_init() was not called on this device */
  QMK_ERR_SIZE = 7,       /* input beyond the allocation-free entry point's limits */
};

/* Device error bits (qmk_device_error). */
enum {
  QMK_DEV_TIMEOUT = 1,    /* a bounded wait expired */
  QMK_DEV_POSITION = 2,   /* persistent-mode position outside the cache */
  QMK_DEV_TOKEN = 4,      /* token id outside the vocabulary */
};

/* One decode step at `position` for `input_token_id`; writes the greedy next
 * token to output_token_id (device int).  Asynchronous on `stream`.
 * Replaces reference csrc/kernel.cu:1477-1505. */
void launch_ldg_decode_direct(
    int input_token_id, int *output_token_id, const void *embed_weight,
    const LDGLayerWeights *layer_weights, const void *final_norm_weight,
    const void *lm_head_weight, const void *cos_table, const void *sin_table,
    void *k_cache, void *v_cache, void *hidden_buffer, void *g_activations,
    void *g_residual, void *g_q, void *g_k, void *g_v, void *g_attn_out,
    void *g_mlp_intermediate, void *g_normalized, void *block_max_vals,
    void *block_max_idxs, int num_layers, int position, int max_seq_len,
    float attn_scale, hipStream_t stream);

/* Same step, but the kernel reads position/token from the stream's device
 * state (set here), the form that a captured graph can replay.  `cache_len`
 * must equal position + 1, as in the reference's only caller convention.
 * Replaces reference csrc/kernel.cu:1507-1543. */
void launch_ldg_decode_persistent(
    int input_token_id, int *output_token_id, const void *embed_weight,
    const LDGLayerWeights *layer_weights, const void *final_norm_weight,
    const void *lm_head_weight, const void *cos_table, const void *sin_table,
    void *k_cache, void *v_cache, void *hidden_buffer, void *g_activations,
    void *g_residual, void *g_q, void *g_k, void *g_v, void *g_attn_out,
    void *g_mlp_intermediate, void *g_normalized, void *block_max_vals,
    void *block_max_idxs, int num_layers, int position, int cache_len,
    int max_seq_len, float attn_scale, hipStream_t stream);

/* num_steps greedy steps starting at start_position with first_token_id,
 * with no host synchronisation between steps: each launch feeds its argmax
 * to the next through device state.  output_log (device int[num_steps])
 * receives the generated tokens.  Asynchronous; the caller synchronises.
 * Replaces reference csrc/kernel.cu:1547-1605. */
void launch_ldg_generate_nosync(
    int first_token_id, int num_steps, const void *embed_weight,
    const LDGLayerWeights *layer_weights, const void *final_norm_weight,
    const void *lm_head_weight, const void *cos_table, const void *sin_table,
    void *k_cache, void *v_cache, void *hidden_buffer, void *g_activations,
    void *g_residual, void *g_q, void *g_k, void *g_v, void *g_attn_out,
    void *g_mlp_intermediate, void *g_normalized, void *block_max_vals,
    void *block_max_idxs, int *output_log, int num_layers, int start_position,
    int max_seq_len, float attn_scale, hipStream_t stream);

/* ---- additions with no counterpart in the reference ---- */

/* Decode step that also writes the fp32 copy of the bf16 logits
 * (float[vocab]) when logits_out is not NULL; used by parity tests.
 * Returns a status code. */
int qmk_decode_logits(
    int input_token_id, int *output_token_id, float *logits_out,
    const void *embed_weight, const LDGLayerWeights *layer_weights,
    const void *final_norm_weight, const void *lm_head_weight,
    const void *cos_table, const void *sin_table, void *k_cache, void *v_cache,
    void *hidden_buffer, void *g_normalized, int num_layers, int position,
    int max_seq_len, float attn_scale, hipStream_t stream);

/* Model shapes for the *_model entry points.  The reference's launchers above
 * serve Qwen3-0.6B, the model the reference is written for. */
enum {
  QMK_MODEL_QWEN3_0_6B = 0, /* 28 layers, hidden 1024, MLP 3072 */
  QMK_MODEL_QWEN3_1_7B = 1, /* 28 layers, hidden 2048, MLP 6144 */
};
/* Both: 16 query heads, 8 KV heads, head_dim 128, vocab 151936, tied LM head;
 * tensors laid out as for the launchers above with the model's dimensions. */

/* One decode step of `model` (and the fp32 copy of its bf16 logits when
 * logits_out is not NULL).  Returns a status code.  Asynchronous. */
int qmk_decode_model(
    int model, int input_token_id, int *output_token_id, float *logits_out,
    const void *embed_weight, const LDGLayerWeights *layer_weights,
    const void *final_norm_weight, const void *lm_head_weight,
    const void *cos_table, const void *sin_table, void *k_cache, void *v_cache,
    void *hidden_buffer, void *g_normalized, int num_layers, int position,
    int max_seq_len, float attn_scale, hipStream_t stream);

/* The library's set-up call for the current device: checks it (gfx950, 256
 * CUs, one decode workgroup per CU) and takes the device address of its copy
 * of the allocation-free entry point's scratch.  Call once per device, with
 * that device current, before qmk_decode_model_noalloc (for example before
 * capturing a graph).  Allocates no device memory.  Returns a status code.
 * No counterpart in the reference. */
int qmk_init(void);

/* qmk_decode_model without any allocation: no hipMalloc, hipFree or other
 * allocating call, on any call.  For callers that cannot allocate: code under
 * HIP graph capture, tight serving loops, harnesses that forbid it.  No
 * counterpart in the reference.
 *
 * The kernel's device state and exchange words live in a file-scope device
 * array of 979,200 bytes per GPU (kept until the process ends) instead of the
 * per-stream buffers the other entry points allocate on first use.  Every call
 * on a GPU shares that array: calls are ordered across streams like every
 * decode launch, but calls replayed from captured graphs on several streams at
 * once race and must not overlap.  Limits: num_layers <= 28 and max_seq_len <=
 * 65536 (QMK_ERR_SIZE beyond them); qmk_init() first (QMK_ERR_INIT).  A call
 * that fails on the device leaves -1 in output_token_id; the next call starts
 * clean.  Returns a status code.  Asynchronous. */
int qmk_decode_model_noalloc(
    int model, int input_token_id, int *output_token_id, float *logits_out,
    const void *embed_weight, const LDGLayerWeights *layer_weights,
    const void *final_norm_weight, const void *lm_head_weight,
    const void *cos_table, const void *sin_table, void *k_cache, void *v_cache,
    void *hidden_buffer, void *g_normalized, int num_layers, int position,
    int max_seq_len, float attn_scale, hipStream_t stream);

/* The allocation-free entry point's status, read without allocating: waits
 * for `stream` and returns the error bits the last qmk_decode_model_noalloc
 * call on the current device left in the scratch array (0 = ok;
 * 0xffffffff if qmk_init() has not run on this device or a HIP call failed).
 * The next qmk_decode_model_noalloc call clears them.  No counterpart in the
 * reference; for the callers that cannot allocate. */
uint32_t qmk_noalloc_device_error(hipStream_t stream);

/* Sets the bound of every device-side wait of qmk_decode_model_noalloc on the
 * current device, in wall-clock ticks (0 restores the default of one second).
 * qmk_init() first (QMK_ERR_INIT).  Tests use a tiny bound to drive its
 * failure path without any risk of a hang.  No counterpart in the reference;
 * for the callers that cannot allocate.  Returns a status code. */
int qmk_noalloc_set_wait_limit(uint32_t ticks);

/* launch_ldg_generate_nosync for `model`.  Returns a status code. */
int qmk_generate_model(
    int model, int first_token_id, int num_steps, const void *embed_weight,
    const LDGLayerWeights *layer_weights, const void *final_norm_weight,
    const void *lm_head_weight, const void *cos_table, const void *sin_table,
    void *k_cache, void *v_cache, void *hidden_buffer, void *g_normalized,
    int *output_log, int num_layers, int start_position, int max_seq_len,
    float attn_scale, hipStream_t stream);

/* qmk_generate_model that stops at a token (the text path's EOS on the
 * device, no counterpart in the reference, which always runs num_steps,
 * csrc/kernel.cu:1547-1605): once a step emits eos_token_id (>= 0), the
 * remaining launches touch no position, cache or exchange and only write
 * eos_token_id into output_log (HF pads finished sequences with
 * pad_token_id = eos_token_id).  The number of generated tokens is the index
 * of the first eos_token_id in output_log plus one (num_steps if absent).
 * Returns a status code.  Asynchronous. */
int qmk_generate_eos(
    int model, int first_token_id, int num_steps, int eos_token_id,
    const void *embed_weight, const LDGLayerWeights *layer_weights,
    const void *final_norm_weight, const void *lm_head_weight,
    const void *cos_table, const void *sin_table, void *k_cache, void *v_cache,
    void *hidden_buffer, void *g_normalized, int *output_log, int num_layers,
    int start_position, int max_seq_len, float attn_scale, hipStream_t stream);

/* ---- sampling (no counterpart in the reference, which is greedy only,
 * csrc/kernel.cu:1020-1183) ----
 * HF's warpers in HF's order: scores s = logit / temperature; top-k keeps
 * s >= the top_k-th largest s (ties kept); top-p keeps a token when the
 * probability mass of the kept scores strictly above it is < top_p (HF removes
 * sorted tokens whose ascending cumulative probability is <= 1 - top_p; the
 * top token always stays); then one draw from the softmax of the kept scores
 * by the Gumbel-max method, argmax of s + G, G = -log(-log(U)), U from the
 * SplitMix64 hash of (seed, counter, token id).  temperature <= 0 is greedy
 * (first index of the maximum); top_k <= 0 or >= vocab and top_p outside
 * (0, 1) switch those filters off.  Same (seed, counter, logits) -> same token.
 */

/* One token per row of logits (float[rows][vocab], device) into out_tokens
 * (int[rows], device); counters (int64[rows], device) give each row its own
 * random numbers.  Asynchronous; returns a status code. */
int qmk_sample_rows(const float *logits, int rows, int vocab, float temperature,
                    int top_k, float top_p, unsigned long long seed,
                    const long long *counters, int *out_tokens, hipStream_t stream);

/* qmk_generate_eos with sampling: every step's greedy token is replaced by a
 * draw from its logits (counter = the step's position) before it is fed to the
 * next step.  eos_token_id < 0: no stop token.  Returns a status code. */
int qmk_generate_sample(
    int model, int first_token_id, int num_steps, int eos_token_id,
    float temperature, int top_k, float top_p, unsigned long long seed,
    const void *embed_weight, const LDGLayerWeights *layer_weights,
    const void *final_norm_weight, const void *lm_head_weight,
    const void *cos_table, const void *sin_table, void *k_cache, void *v_cache,
    void *hidden_buffer, void *g_normalized, int *output_log, int num_layers,
    int start_position, int max_seq_len, float attn_scale, hipStream_t stream);

/* The generate entry points record 32 persistent launches into a HIP graph
 * once per stream and argument set and replay it (the remainder is launched
 * directly); enable = 0 launches every step directly, as the reference's loop
 * does (csrc/kernel.cu:1584-1600).  Default on.  Returns a status code. */
int qmk_set_graph_launch(hipStream_t stream, int enable);

/* Status of the last call made on this thread. */
int qmk_last_status(void);
const char *qmk_status_string(int status);

/* Synchronises `stream` and returns its latched device error bits (0 = ok). */
uint32_t qmk_device_error(hipStream_t stream);

/* Clears the stream's device state (error bits, exchange buffers).
 * Synchronous.  Returns a status code. */
int qmk_reset(hipStream_t stream);

/* Sets the bound of every device-side wait for launches on `stream`, in
 * wall-clock ticks (0 restores the default of one second).  Tests use a tiny
 * bound to drive the failure path without any risk of a hang. */
int qmk_set_wait_limit(hipStream_t stream, uint32_t ticks);

/* Phase trace.  When `buf` (device uint64[qmk_trace_entries(28)]) is set,
 * every launch on `stream` writes, for each workgroup w, the 100 MHz device
 * wall clock at 13 points of each layer and 3 points after the last layer:
 * buf[point * 256 + w], point = layer * 13 + k; then compute wave 0 writes
 * the start and end of its 6 phases per layer at
 * buf[(num_layers*13 + 3 + layer*12 + k) * 256 + w].  NULL disables tracing. */
int qmk_set_trace(hipStream_t stream, uint64_t *buf, size_t entries);
size_t qmk_trace_entries(int num_layers);

/* Runs the decode kernel's arithmetic building blocks on one wave so tests can
 * check them: out[0,n) = bf16 rounding of in[i], out[n,2n) = the softmax exp
 * of in[i], out[2n + 64k + lane] for k = 0..4: sum over the four 16-lane rows,
 * then the two results of the row-pair swap and of the half-wave swap of
 * in[lane].  n >= 64; out holds 2n + 320 floats.  Asynchronous. */
int qmk_selftest_blocks(const float *in, float *out, int n, hipStream_t stream);

/* Per-phase weight-streaming microbenchmark.  Runs one GEMV phase of the
 * decode step over n_copies distinct weight copies laid out one after another
 * (qmk_phase_copy_elems(phase) bf16 elements each), with the decode kernel's
 * work split and one-copy-ahead prefetch, so the phase's HBM rate can be
 * measured on its own.  Phases:
 *   0 QKV      RMSNorm(act[1024], norm_weight) then [4096][1024] (q, k, v rows);
 *              out bf16[4096]
 *   1 O        [1024][2048] x act[2048]; out f32[8][1024] per-XCD partial sums
 *              over input columns [256x, 256x+256)
 *   2 GATE_UP  gate [3072][1024] then up [3072][1024] x act[1024];
 *              out bf16[3072] = bf16(bf16(silu(g)) * u)
 *   3 DOWN     [1024][3072] x act[3072]; out f32[8][1024] partials over
 *              columns [384x, 384x+384)
 *   4 LM_HEAD  [151936][1024] x act[1024]; out uint64[256*8] per-wave best
 *              keys (orderable bf16 logit << 32 | ~row): the largest key is
 *              the argmax
 * out holds the last copy's results.  Asynchronous; returns a status code. */
int qmk_phase_bench(int phase, const void *weights, int n_copies,
                    const void *norm_weight, const void *act, void *out,
                    hipStream_t stream);
size_t qmk_phase_copy_elems(int phase);

/* Kernel launch geometry, for tools: workgroups and threads per workgroup. */
void qmk_launch_geometry(int *workgroups, int *threads);

/* ---- batched forward (no counterpart in the reference, which feeds a
 * prompt one decode step per token, qwen_megakernel/model.py:207-211) ---- */

/* Workspace bytes qmk_forward_tokens needs for `num_tokens` tokens,
 * `num_emit` emitted rows (<= 256) and contexts of at most `max_context`
 * positions.  0 for invalid arguments. */
size_t qmk_forward_workspace_bytes(int model, int num_tokens, int num_emit,
                                   int max_context);

/* One forward pass of `num_tokens` tokens through `model`, on MFMA GEMMs
 * (one weight read serves every token).  Token t is token id tokens[t] of
 * sequence seq_ids[t] at position positions[t]: its K/V are written into that
 * sequence's cache at that position, and it attends to positions
 * 0..positions[t] of the sequence, so the tokens of one sequence at
 * consecutive positions form a prompt prefill (causal), and one token per
 * sequence a batched decode step.  Sequence s's cache is the
 * [num_layers][8][max_seq_len][128] block at k_cache + s * seq_stride
 * (elements; seq_stride is ignored when num_seqs == 1).  For the emitted rows
 * e = emit_rows[r] (r < num_emit), out_tokens[r] receives the greedy next
 * token after token e and, when logits_out is not NULL, logits_out[r][vocab]
 * the fp32 copy of its bf16 logits.  A token with an id outside the
 * vocabulary, a sequence outside [0, num_seqs) or a position outside
 * [0, max_context) writes no cache and emits -1; so does an emit row outside
 * [0, num_tokens).  tokens, seq_ids, positions, emit_rows, out_tokens and
 * logits_out are device pointers; layer_weights_host is a HOST array of
 * num_layers tables (device pointers inside).  max_context <= max_seq_len
 * bounds every position + 1 (it sizes the workspace).  Asynchronous; returns
 * a status code. */
int qmk_forward_tokens(
    int model, int num_tokens, const int *tokens, const int *seq_ids,
    const int *positions, int num_emit, const int *emit_rows, int *out_tokens,
    float *logits_out, const void *embed_weight,
    const LDGLayerWeights *layer_weights_host, const void *final_norm_weight,
    const void *lm_head_weight, const void *cos_table, const void *sin_table,
    void *k_cache, void *v_cache, int num_seqs, long long seq_stride,
    int num_layers, int max_seq_len, int max_context, float attn_scale,
    void *workspace, size_t workspace_bytes, hipStream_t stream);

/* Workspace bytes qmk_decode_batch needs.  0 for invalid arguments. */
size_t qmk_decode_batch_workspace_bytes(int model, int batch, int max_context);

/* One batched decode step: token b (tokens[b], device) of sequence b at
 * positions[b] (device), b < batch; out_tokens[b] (device) receives its greedy
 * next token, logits_out[b][vocab] its logits when not NULL.  Sequence b's
 * cache is the [num_layers][8][max_seq_len][128] block at k_cache + b *
 * seq_stride.  The same as qmk_forward_tokens with seq_ids = emit_rows =
 * 0..batch-1, but since each sequence has one token, batches of up to 16 with
 * max_context <= 4096 run five fused launches per layer (RMSNorm in the GEMM
 * prologues, q/k norm + RoPE + K/V append inside attention, residual and
 * SiLU*up in the GEMM epilogues).  Invalid ids or positions emit -1.
 * tokens and positions may share memory with out_tokens (an in-place step):
 * such calls take the multi-launch path, which reads them before writing.
 * Asynchronous; returns a status code. */
int qmk_decode_batch(
    int model, int batch, const int *tokens, const int *positions, int *out_tokens,
    float *logits_out, const void *embed_weight,
    const LDGLayerWeights *layer_weights_host, const void *final_norm_weight,
    const void *lm_head_weight, const void *cos_table, const void *sin_table,
    void *k_cache, void *v_cache, long long seq_stride, int num_layers,
    int max_seq_len, int max_context, float attn_scale, void *workspace,
    size_t workspace_bytes, hipStream_t stream);

/* The batched decode step of qmk_decode_batch as one persistent kernel
 * launch: the arguments and results of qmk_decode_batch (no workspace), for
 * 2 <= batch <= 4 and max_context <= 2048.  The 256 workgroups of the decode
 * kernel stream each weight slice once and apply it to all `batch` rows;
 * activations move between workgroups through the per-stream exchange area
 * (allocated on the stream's first call).  The layer table is copied to
 * device memory once per distinct table (up to 64 per device, kept until the
 * process ends).  tokens and positions must not overlap out_tokens, which
 * receives -1 first, so a step that fails on the device (qmk_device_error)
 * leaves -1 (QMK_ERR_ARG otherwise).  Returns QMK_ERR_DEVICE where the kernel
 * does not fit one workgroup per CU, or where a new table cannot be copied
 * now (the stream is being captured, or 64 tables are kept);
 * qmk_decode_batch then keeps its multi-launch path.  No counterpart in the
 * reference, which decodes one sequence (qwen_megakernel/model.py:111-250).
 * Asynchronous. */
int qmk_decode_batch_persistent(
    int model, int batch, const int *tokens, const int *positions, int *out_tokens,
    float *logits_out, const void *embed_weight,
    const LDGLayerWeights *layer_weights_host, const void *final_norm_weight,
    const void *lm_head_weight, const void *cos_table, const void *sin_table,
    void *k_cache, void *v_cache, long long seq_stride, int num_layers,
    int max_seq_len, int max_context, float attn_scale, hipStream_t stream);

/* Process-wide switch (default on): qmk_decode_batch runs the persistent
 * kernel above for the shapes it covers.  Off: always the multi-launch path
 * (for comparisons).  Returns QMK_OK. */
int qmk_set_batch_persistent(int enable);

/* 1 while qmk_decode_batch uses the persistent kernel where it applies. */
int qmk_batch_persistent_enabled(void);

/* One 16x16x32 bf16 MFMA with the operand layouts the batched GEMM assumes:
 * c[16][16] (f32) = a[16][32] . b[16][32]^T (bf16, row-major).  For tests.
 * Asynchronous; returns a status code. */
int qmk_selftest_mfma(const void *a, const void *b, float *c, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* QWEN_MEGAKERNEL_AMD_H */
