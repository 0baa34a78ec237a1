/*
 * rtq.h — C ABI of the MI355X (gfx950) frozen quantised-matmul library (librtq.so).
 *
 * Drop-in boundary for Rust_Trainer's frozen-weight plugin point:
 *   trait FrozenMatmul            src/frozen.rs:14-25  (out_dim, in_dim, forward, backward_input, row, nbytes)
 *   impl FrozenMatmul for RieFrozen  src/rie.rs:66-129 (the engine-backed GGUF implementation this replaces)
 *   RieFrozen::new / loader `fz`  src/rie.rs:58-60, :183 (constructed from a GGUF Weight's packed bytes)
 *   Linear::forward / backward    src/linear.rs:73-121 (the LoRA math above the frozen weight)
 *
 * Conventions (mirroring the reference):
 *   - all matrices are row-major f32; a weight is [rows = out x cols = in] in GGUF block format;
 *   - forward OVERWRITES y; backward_input ACCUMULATES into dx (dx += dy . W);
 *     linear_backward returns a fresh dx (overwrites) and ACCUMULATES ga / gb;
 *   - errors are status codes (the reference asserts; a Rust wrapper panics on non-zero);
 *   - host-pointer entry points are synchronous (they run on the context's own stream); `_d` entry
 *     points take device pointers and a HIP stream (hipStream_t passed as void*, NULL = the HIP
 *     null stream, as torch's default stream is) and only enqueue.
 *     Calls on one context are serialised by a lock; `_d` calls that share a context must be
 *     issued on one stream (they share the context's device workspace).
 */
#ifndef RTQ_H
#define RTQ_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int rtq_status;
#define RTQ_OK 0
#define RTQ_ERR_INVALID 1     /* bad argument / shape mismatch (reference: assert!) */
#define RTQ_ERR_UNSUPPORTED 2 /* weight type other than Q4_0, Q8_0, Q4_K, Q6_K, F32, TQ8_0 */
#define RTQ_ERR_HIP 3         /* HIP runtime error (message in rtq_last_error) */
#define RTQ_ERR_NO_DEVICE 4   /* no usable gfx950 device / code object failed to load */

/* GGUF / ggml type ids accepted by rtq_weight_create */
#define RTQ_TYPE_Q4_0 2
#define RTQ_TYPE_Q8_0 8
#define RTQ_TYPE_Q4_K 12
#define RTQ_TYPE_Q6_K 14
/* The trainer-native FrozenWeight storage (src/frozen.rs:33-45, HF / random-init models):
 *   F32:   row-major f32 [rows x cols] (ggml id 0);
 *   TQ8_0: not a ggml type - FrozenWeight::Q8_0, an f32 scale per 32 elements: the scales
 *          [rows x cols/32] (f32) followed by the codes [rows x cols] (i8), cols % 32 == 0.
 * Their forward takes f32 activations (no activation quantisation) and runs as f32 GEMMs. */
#define RTQ_TYPE_F32 0
#define RTQ_TYPE_TQ8_0 264

typedef struct rtq_ctx rtq_ctx;
typedef struct rtq_weight rtq_weight;
typedef struct rtq_gguf rtq_gguf; /* GGUF v3 image (reader, below) */

/* LoRA adapter view (src/linear.rs:8-16): a is [rank x in], b is [out x rank], scale = alpha/rank.
 * enabled = 0 bypasses the adapter (Linear::lora_enabled, src/linear.rs:45). */
typedef struct rtq_lora {
  int64_t rank;
  float alpha;
  const float* a;
  const float* b;
  int enabled;
} rtq_lora;

/* ---- library / context ---- */
const char* rtq_version(void);
const char* rtq_last_error(void); /* thread-local message of the last failing call */
/* Opens device `device`, loads the embedded gfx950 code object (hipModuleLoadData), creates a stream.
 * Replaces the engine ThreadPool the reference threads through RieFrozen (src/rie.rs:53,182). */
rtq_status rtq_ctx_create(int device, rtq_ctx** out);
void rtq_ctx_destroy(rtq_ctx* ctx);
void* rtq_ctx_stream(rtq_ctx* ctx); /* the context's hipStream_t */
/* Pre-sizes the device workspace for calls up to t tokens on any weight of this context. */
rtq_status rtq_ctx_reserve(rtq_ctx* ctx, int64_t max_t, int64_t max_rows, int64_t max_cols, int64_t max_rank);
/* Per-kernel timing with HIP events recorded around launches (off by default); only_kernel (may be
 * NULL) restricts the events to launches of the kernel with that name. */
rtq_status rtq_ctx_set_timing(rtq_ctx* ctx, int enable, const char* only_kernel);
/* Synchronises, folds the recorded events into per-kernel totals, returns the number of kernels seen. */
int rtq_ctx_timing_count(rtq_ctx* ctx);
rtq_status rtq_ctx_timing_get(rtq_ctx* ctx, int i, const char** name, int64_t* launches, double* total_ms);
/* the algorithmic work of kernel i's timed launches (frozen-linear GEMM / GEMV and dx kernels; 0
 * for others): flops 2 T N K (+ the LoRA products in the forward) and bytes = GGUF weight bytes +
 * f32 inputs and outputs (+ A, B), each operand counted once */
rtq_status rtq_ctx_timing_work(rtq_ctx* ctx, int i, double* flops, double* bytes);
void rtq_ctx_timing_reset(rtq_ctx* ctx);

/* ---- weights (RieFrozen::new, src/rie.rs:58-60; Weight::data() bytes, src/rie.rs:186) ---- */
/* blocks: rows * row_bytes(type, cols) bytes of GGUF blocks on the host; uploaded once into the
 * device fragment layout (same byte count, padded to 64-row / 128|256-column tiles). */
rtq_status rtq_weight_create(rtq_ctx* ctx, int ggml_type, const void* blocks, size_t nbytes, int64_t rows,
                             int64_t cols, rtq_weight** out);
void rtq_weight_destroy(rtq_weight* w);
int64_t rtq_weight_out_dim(const rtq_weight* w); /* FrozenMatmul::out_dim, src/frozen.rs:15 */
int64_t rtq_weight_in_dim(const rtq_weight* w);  /* FrozenMatmul::in_dim,  src/frozen.rs:16 */
size_t rtq_weight_nbytes(const rtq_weight* w);   /* FrozenMatmul::nbytes (GGUF bytes), src/frozen.rs:24 */
int rtq_weight_type(const rtq_weight* w);

/* ---- FrozenMatmul (host pointers, synchronous) ---- */
/* y[t x out] = x[t x in] . W^T    (src/frozen.rs:17-18; RieFrozen::forward src/rie.rs:74-82) */
rtq_status rtq_frozen_forward(rtq_ctx* ctx, const rtq_weight* w, const float* x, int64_t t, float* y);
/* dx[t x in] += dy[t x out] . W   (src/frozen.rs:19-20; RieFrozen::backward_input src/rie.rs:84-120) */
rtq_status rtq_frozen_backward_input(rtq_ctx* ctx, const rtq_weight* w, const float* dy, int64_t t, float* dx);
/* out[in] = dequant(W[r])          (src/frozen.rs:21-22; RieFrozen::row src/rie.rs:122-124) */
rtq_status rtq_frozen_row(rtq_ctx* ctx, const rtq_weight* w, int64_t r, float* out);

/* ---- Linear (host pointers, synchronous) ---- */
/* y = x.W^T (+ bias) (+ (alpha/r) (x.A^T).B^T)     (Linear::forward, src/linear.rs:73-93) */
rtq_status rtq_linear_forward(rtq_ctx* ctx, const rtq_weight* w, const float* bias, const rtq_lora* lora,
                              const float* x, int64_t t, float* y);
/* dx = dy.W (+ s (dy.B).A); ga += (s dy.B)^T x; gb += (s dy)^T (x.A^T)   (Linear::backward, src/linear.rs:97-121) */
rtq_status rtq_linear_backward(rtq_ctx* ctx, const rtq_weight* w, const rtq_lora* lora, const float* x,
                               const float* dy, int64_t t, float* dx, float* ga, float* gb);

/* ---- device-pointer variants (enqueue only; same semantics) ---- */
rtq_status rtq_frozen_forward_d(rtq_ctx* ctx, const rtq_weight* w, const float* x, int64_t t, float* y, void* stream);
rtq_status rtq_frozen_backward_input_d(rtq_ctx* ctx, const rtq_weight* w, const float* dy, int64_t t, float* dx,
                                       void* stream);
rtq_status rtq_frozen_rows_d(rtq_ctx* ctx, const rtq_weight* w, int64_t r0, int64_t count, float* out, void* stream);
/* lora->a / lora->b and bias are device pointers here */
rtq_status rtq_linear_forward_d(rtq_ctx* ctx, const rtq_weight* w, const float* bias, const rtq_lora* lora,
                                const float* x, int64_t t, float* y, void* stream);
rtq_status rtq_linear_backward_d(rtq_ctx* ctx, const rtq_weight* w, const rtq_lora* lora, const float* x,
                                 const float* dy, int64_t t, float* dx, float* ga, float* gb, void* stream);

/* rtq_linear_forward_d that allocates nothing.  No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Its workspace is a 64 MiB device array of the library, one per GPU, held
 * from the first context on that GPU until the process ends; a call whose workspace would exceed it
 * fails with RTQ_ERR_INVALID before launching anything (config 1, 256 tokens over 3072 x 1024, needs
 * 0.8 MiB; 2048 tokens over K = 4096 about 19 MiB).  Every call on one GPU shares that array, so
 * calls that overlap on one GPU (other streams, other contexts, other threads) race; calls on one
 * stream do not. */
rtq_status rtq_linear_forward_noalloc_d(rtq_ctx* ctx, const rtq_weight* w, const float* bias, const rtq_lora* lora,
                                        const float* x, int64_t t, float* y, void* stream);

/* ---- embedding gather and LM head + cross-entropy ---- */
/* embed_tokens (src/model.rs:446-454): out[i x in] = row(ids[i]).  Host version: ids out of range are
 * rejected (the reference asserts, :450); device version: such rows come out NaN, nothing is read. */
rtq_status rtq_frozen_gather(rtq_ctx* ctx, const rtq_weight* w, const int32_t* ids, int64_t count, float* out);
rtq_status rtq_frozen_gather_d(rtq_ctx* ctx, const rtq_weight* w, const int32_t* ids, int64_t count, float* out,
                               void* stream);
/* Model::head (src/model.rs:561-609) for n targets (pos[i] < t, tok[i] < vocab = lm_head rows):
 * ns = rmsnorm(x[pos], norm_w, eps, offset) (src/ops.rs:14-36), logits = lm_head.forward(ns),
 * softmax_row with an f64 normaliser (src/ops.rs:238-247), logp[i] = logit[tok] - lse, a hit when
 * the target's logit is >= every logit.  With weights (else NULL, and dx unused): for
 * L = -sum weights[i] logp[i], dx[t x d] = dL/dx, OVERWRITTEN (zero outside target rows;
 * targets sharing a position add in target order).  All targets are processed in one pass (the
 * reference's 64-target chunks bound its memory; here the workspace holds n x vocab logits).
 * Host version: *hits = number of hits, targets out of range rejected.  Device version: hit[i]
 * per target (0 / 1); a target out of range reads nothing and gets logp NaN, hit 0, no gradient. */
rtq_status rtq_lm_head(rtq_ctx* ctx, const rtq_weight* lm_head, const float* norm_w, float eps, float offset,
                       const float* x, int64_t t, const int32_t* pos, const int32_t* tok, const float* weights,
                       int64_t n, float* logp, int64_t* hits, float* dx);
rtq_status rtq_lm_head_d(rtq_ctx* ctx, const rtq_weight* lm_head, const float* norm_w, float eps, float offset,
                         const float* x, int64_t t, const int32_t* pos, const int32_t* tok, const float* weights,
                         int64_t n, float* logp, int32_t* hit, float* dx, void* stream);

/* ---- device-resident training step (Model::forward_backward over the frozen linears) ----
 * A GGUF Qwen / Llama decoder (load_gguf_from, src/rie.rs:164-260) with every frozen tensor, norm
 * and adapter in device memory.  One call runs embed_tokens, the blocks (RMSNorm, q/k/v, QK-norm,
 * RoPE, f16 K/V, causal GQA attention, o, SwiGLU MLP: src/model.rs:165-197, src/attention.rs:
 * 162-367, src/model.rs:113-134), Model::head and the blocks' backward in reverse
 * (src/model.rs:644-687), accumulating the adapters' gradients on the device.  Every block's
 * activations are kept for its backward instead of being recomputed (the same values). */
typedef struct rtq_model rtq_model;
typedef struct rtq_model_config {
  int64_t n_layer, n_embd, n_head, n_head_kv, head_dim, rope_dim, n_ff, n_vocab;
  float rms_eps, norm_offset, rope_base, rope_freq_scale;
  int rope_neox, qk_norm, kv_f16, tied;
  int64_t n_rope_factors; /* length of rope_freqs.weight (0: none) */
} rtq_model_config;
/* hyper-parameters from `<arch>.*` keys, tensors blk.{i}.{attn_q,attn_k,attn_v,attn_output,
 * ffn_gate,ffn_up,ffn_down}.weight (+ optional q/k/v .bias), norms F32; tied when output.weight is
 * absent.  Refused with RTQ_ERR_UNSUPPORTED as the reference's loader refuses them: architectures
 * other than llama / qwen2 / qwen3 (trainable_arch, src/rie.rs:153-155), embedding / residual /
 * logit scales other than 1, softcaps, a sliding window, an attention scale other than
 * 1/sqrt(head_dim) (src/rie.rs:173-183), mixture-of-experts FFNs (:211-216), post-norm layers
 * (:204-206), and RoPE scaling other than none / linear.  Linear RoPE scaling
 * (<arch>.rope.scaling.factor) and rope_freqs.weight (per-frequency divisors) are applied as
 * Rope::at_positions does (src/ops.rs:141-158). */
rtq_status rtq_model_from_gguf(rtq_ctx* ctx, const rtq_gguf* g, rtq_model** out);
/* the hyper-parameters and refusals of rtq_model_from_gguf alone, without a device */
rtq_status rtq_model_config_from_gguf(const rtq_gguf* g, rtq_model_config* out);
void rtq_model_destroy(rtq_model* m);
rtq_status rtq_model_get_config(const rtq_model* m, rtq_model_config* out);
/* Model::attach_lora (src/model.rs:406-419): target_mask bit i adapts linear i of (q, k, v, o, gate,
 * up, down) in every block; A ~ U(-1/sqrt(in), 1/sqrt(in)) drawn from Rng(seed) in block order, B = 0
 * (Lora::new, src/linear.rs:21-25); *n_params = adapter parameters */
rtq_status rtq_model_attach_lora(rtq_model* m, int64_t rank, float alpha, uint32_t target_mask, uint64_t seed,
                                 int64_t* n_params);
int64_t rtq_model_lora_count(const rtq_model* m); /* adapted linears, in (block, q..down) order */
rtq_status rtq_model_lora_info(const rtq_model* m, int64_t i, int* layer, int* which, int64_t* rank, int64_t* in,
                               int64_t* out, float* alpha);
/* host copies of adapter i's a [rank x in], b [out x rank], ga, gb (any may be NULL) */
rtq_status rtq_model_lora_get(rtq_model* m, int64_t i, float* a, float* b, float* ga, float* gb);
rtq_status rtq_model_lora_set(rtq_model* m, int64_t i, const float* a, const float* b);
/* device pointers of adapter i (an optimiser on the device updates a / b in place): a, ga are
 * [rank x in] contiguous; b, gb are [out x rank] blocks with row stride *ldb floats (adapters of
 * linears that run fused share one matrix) */
rtq_status rtq_model_lora_device(rtq_model* m, int64_t i, float** a, float** b, float** ga, float** gb, int64_t* ldb);
rtq_status rtq_model_zero_grad(rtq_model* m); /* Model::zero_grad (src/model.rs:436) */
/* Model::forward_backward (src/model.rs:615-687) on one sequence (host arrays): tokens [t], targets
 * (pos[i], tok[i]) with loss weights [n]; logp [n] and *hits out.  weights NULL: log-probs only
 * (Model::score, no backward).  Synchronous on the context's stream. */
rtq_status rtq_model_forward_backward(rtq_model* m, const int32_t* tokens, int64_t t, const int32_t* pos,
                                      const int32_t* tok, const float* weights, int64_t n, float* logp,
                                      int64_t* hits);
/* Model::forward_backward_packed (src/model.rs:634-642) on a packed batch (Packed / pack,
 * src/model.rs:234-290): positions [t] (RoPE, Model::rope_for :461-481) and segments [t] of every
 * token; token i may attend to token j <= i when segments[j] is 0 (the shared prompt) or equals
 * segments[i] (Rope::allowed, src/ops.rs:160-167).  Targets index the packed tokens. */
rtq_status rtq_model_forward_backward_packed(rtq_model* m, const int32_t* tokens, int64_t t,
                                             const int32_t* positions, const int32_t* segments, const int32_t* pos,
                                             const int32_t* tok, const float* weights, int64_t n, float* logp,
                                             int64_t* hits);
/* Model::checkpointing (src/model.rs:299-300; the loader's default true, src/rie.rs:254): 1 keeps
 * only each block's input and recomputes its forward in the backward (src/model.rs:663-665,
 * 678-680); 0 keeps every block's activations; -1 (default) keeps them when they take at most half
 * of the device memory free at the step, else recomputes.  The results are the same. */
rtq_status rtq_model_set_checkpointing(rtq_model* m, int mode);
int rtq_model_checkpointing(const rtq_model* m); /* 1 when the last step recomputed */
/* Attention kernels of the step (the results agree within f32 rounding): 1 the fused kernels
 * (online softmax, no probability matrix; head_dim 64 or 128 only), 0 the probability-matrix path
 * (S, softmax, P V and their backward as separate launches, P [heads x t x t] kept per layer), -1
 * (default) fused whenever the head size allows. */
rtq_status rtq_model_set_attention(rtq_model* m, int mode);
int rtq_model_attention_fused(const rtq_model* m); /* 1 when the last step used the fused kernels */
/* Steps run as one HIP graph where they can: a step whose launch key (t, n, with or without
 * weights, the packed layout, the checkpointing and attention choices, adapters and buffers) equals
 * the previous step's is captured, and later steps with that key replay it; the inputs' upload and
 * the outputs' download stay outside.  RTQ_STEP_GRAPH=0 in the environment when the model is
 * loaded keeps every step eager.  No counterpart in the reference (its steps are eager host code):
 * the number of replays so far, for tests and profiling. */
int64_t rtq_model_graph_replays(const rtq_model* m);
/* parity / debug: while layer >= 0 (-1: off), each step copies that block's tensors in the forward
 * (x, n1, inv1, q_raw, k_raw, v_raw, q, k, v, q_inv, k_inv, P [nh x t x t], o, h, n2, inv2, gate,
 * up, hm, y) and its backward (dy, dhm, dgate, dup, dn2, dh, d_o, dS, dq, dk, dv, dq_raw, dk_raw,
 * dn1, dx), row-major per token; rtq_model_debug_tensor copies one to the host (nfloats must match;
 * out NULL: only checks that the tensor exists and holds at most nfloats). */
rtq_status rtq_model_debug_capture(rtq_model* m, int64_t layer);
rtq_status rtq_model_debug_tensor(rtq_model* m, const char* name, float* out, int64_t nfloats);

/* ---- parity / debug (host pointers, synchronous) ---- */
/* The activation blocks the GPU forward actually uses for x, in ggml layout (block_q8_0: 34 B per
 * 32 elements for Q4_0/Q8_0 weights; block_q8_K: 292 B per 256 for Q4_K/Q6_K), t * act_row_bytes. */
rtq_status rtq_debug_quantize_acts(rtq_ctx* ctx, const rtq_weight* w, const float* x, int64_t t, void* out);
int64_t rtq_debug_isums_per_row(const rtq_weight* w);
/* The integer block sums computed by the GPU forward kernel itself: int32 [t][out][isums_per_row]
 * (Q4_0/Q8_0: one per 32-block; Q4_K: (S1, S2) per super-block; Q6_K: S per super-block). */
rtq_status rtq_debug_block_isums(rtq_ctx* ctx, const rtq_weight* w, const float* x, int64_t t, int32_t* out);

/* ---- GGUF v3 container (rie_core::gguf::{GgufFile, GgufWriter}) ----
 * Reader: GgufFile::open (src/rie.rs:159, :370) maps the file; GgufFile::from_bytes
 * (tests/engine.rs:27-31, examples/bench_train.rs:28-32, tests/agentd.rs:14) borrows the caller's bytes, which must
 * outlive the handle.  Every length and offset is checked against the image (RTQ_ERR_INVALID with
 * a message otherwise).  Strings and tensor data point into the image; they are valid until close.
 * Value types: u8 0, i8 1, u16 2, i16 3, u32 4, i32 5, f32 6, bool 7, string 8, array 9, u64 10,
 * i64 11, f64 12.  Tensor dims ne[0] = row length (columns), ne[1..] = rows (n_rows/row_len). */
typedef struct rtq_gguf_writer rtq_gguf_writer;
rtq_status rtq_gguf_open(const char* path, rtq_gguf** out);
rtq_status rtq_gguf_from_bytes(const void* data, size_t nbytes, rtq_gguf** out);
void rtq_gguf_close(rtq_gguf* g);
uint32_t rtq_gguf_version(const rtq_gguf* g);
int64_t rtq_gguf_kv_count(const rtq_gguf* g);
int64_t rtq_gguf_find_kv(const rtq_gguf* g, const char* key); /* -1 if absent */
/* key i: type, array element type (-1 unless an array), count (array length / string bytes / 1),
 * data (the value; arrays of strings: the first u64-length-prefixed element) */
rtq_status rtq_gguf_kv(const rtq_gguf* g, int64_t i, const char** key, int* type, int* elem_type, uint64_t* count,
                       const void** data);
/* GgufFile::get_str (src/rie.rs:371-374): not NUL-terminated, length in *len */
rtq_status rtq_gguf_get_str(const rtq_gguf* g, const char* key, const char** s, uint64_t* len);
/* GgufFile::get_f32 / get_u32 (src/rie.rs:379): any numeric or bool value, widened to double */
rtq_status rtq_gguf_get_f64(const rtq_gguf* g, const char* key, double* v);
int64_t rtq_gguf_tensor_count(const rtq_gguf* g);
int64_t rtq_gguf_find_tensor(const rtq_gguf* g, const char* name); /* GgufFile::tensor; -1 if absent */
/* GgufFile::tensor + tensor_data (src/rie.rs:381-384): nbytes is 0 for a ggml type of unknown size */
rtq_status rtq_gguf_tensor(const rtq_gguf* g, int64_t i, const char** name, int* type, int* n_dims, int64_t ne[4],
                           const void** data, size_t* nbytes);
/* Uploads a GGUF tensor as a frozen weight (the loader's `fz(ggml type, bytes, rows, cols)`,
 * src/rie.rs:183-190): rows = ne[1]*ne[2]*ne[3], cols = ne[0]. */
rtq_status rtq_weight_from_gguf(rtq_ctx* ctx, const rtq_gguf* g, const char* name, rtq_weight** out);

/* Writer (GgufWriter::new / kv / tensor / to_bytes, src/rie.rs:349-363).  Tensors are laid out in
 * insertion order at general.alignment (default 32; set it as a u32 key before writing). */
rtq_status rtq_gguf_writer_create(rtq_gguf_writer** out);
void rtq_gguf_writer_destroy(rtq_gguf_writer* w);
/* scalar: count 1, data -> the value; string (8): count bytes at data; array (9): count elements of
 * elem_type at data (an array of strings: data is const char* const*, NUL-terminated strings) */
rtq_status rtq_gguf_writer_kv(rtq_gguf_writer* w, const char* key, int type, int elem_type, uint64_t count,
                              const void* data);
/* nbytes must be the ggml size of ne[0]*...*ne[n_dims-1] elements of type */
rtq_status rtq_gguf_writer_tensor(rtq_gguf_writer* w, const char* name, int type, int n_dims, const int64_t* ne,
                                  const void* data, size_t nbytes);
/* the image (to_bytes), owned by the writer until its next call or destroy */
rtq_status rtq_gguf_writer_bytes(rtq_gguf_writer* w, const void** data, size_t* nbytes);
/* the image written to path.tmp, then renamed to path (src/rie.rs:359-362) */
rtq_status rtq_gguf_writer_write(rtq_gguf_writer* w, const char* path);

#ifdef __cplusplus
}
#endif
#endif
