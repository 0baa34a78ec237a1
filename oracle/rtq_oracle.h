/*
 * rtq_oracle.h — CPU restatement of Rust_Trainer's frozen quantised-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the checker / the timed CPU
 * baseline.  The product path (librtq.so) never links or calls it.
 *
 * Reference sources restated (files under the reference repository):
 *   src/frozen.rs:14-25     FrozenMatmul contract (forward overwrites y, backward_input accumulates dx)
 *   src/rie.rs:74-82        RieFrozen::forward   = activation quantisation + integer block dots
 *   src/rie.rs:84-120       RieFrozen::backward_input = 32-row dequant chunks + f32 axpy, reduced
 *   src/rie.rs:122-124      RieFrozen::row       = Weight::dequant_row
 *   src/linear.rs:73-121    Linear::forward / Linear::backward (LoRA order)
 *   src/tensor.rs:24-120    dot / axpy / matmul_nt / matmul_nn / matmul_tn_acc
 *   src/tensor.rs:155-199   Rng (SplitMix64 + Box-Muller)
 *   src/model.rs:561-609    Model::head (final RMSNorm, LM head, log-softmax, dlogits, RMSNorm backward)
 *   ggml block formats Q4_0, Q8_0, Q4_K, Q6_K and activation blocks Q8_0 / Q8_K; rie-core
 *   (git dependency pinned at f3be365b41f929cc81ee08afaa994d02bbeee2f5, Cargo.lock:529-540,
 *   absent from the container) follows ggml's public block semantics for these formats.
 */
#ifndef RTQ_ORACLE_H
#define RTQ_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (same numbering as the GGUF format) */
enum {
  OR_F32 = 0,
  OR_F16 = 1,
  OR_Q4_0 = 2,
  OR_Q8_0 = 8,
  OR_Q4_K = 12,
  OR_Q6_K = 14,
  OR_Q8_K = 15,
  /* not a ggml type: the trainer-native FrozenWeight::Q8_0 (src/frozen.rs:38-45), f32 scale per 32
     elements; packed as the scales [n][k/32] (f32) followed by the codes [n][k] (i8) */
  OR_TQ8_0 = 264
};

/* ---- trainer-native FrozenWeight::Q8_0 (src/frozen.rs:53-73 quantiser, :80-108 dot / axpy) ---- */
int or_tq8_quantize(const float* w, int64_t n, int64_t k, void* out);

/* ---- Rng: src/tensor.rs:155-199 ---- */
uint64_t or_rng_seed(uint64_t seed);
uint64_t or_rng_next_u64(uint64_t* state);
float or_rng_uniform(uint64_t* state);
float or_rng_normal(uint64_t* state);
void or_rng_fill_normal(uint64_t* state, float* out, int64_t n, float std);
void or_rng_fill_uniform_sym(uint64_t* state, float* out, int64_t n, float bound);

/* ---- IEEE half ---- */
uint16_t or_fp32_to_fp16(float f);
float or_fp16_to_fp32(uint16_t h);

/* ---- block formats ---- */
int64_t or_block_elems(int type);
int64_t or_block_bytes(int type);
int64_t or_row_bytes(int type, int64_t k);
/* weight quantisers; n must be a multiple of the block size */
int or_quantize(int type, const float* x, int64_t n, void* out);
/* one row of k elements -> f32; returns 0 on success */
int or_dequant_row(int type, const void* row, int64_t k, float* out);

/* ---- activation quantisation (QuantActs::prepare, src/rie.rs:77-78) ---- */
/* act type paired with a weight type: Q8_0 for Q4_0/Q8_0, Q8_K for Q4_K/Q6_K, F32 otherwise */
int or_act_type_for(int wtype);
void or_quantize_acts_q8_0(const float* x, int64_t k, void* out); /* k % 32 == 0, 34 B blocks */
void or_quantize_acts_q8_k(const float* x, int64_t k, void* out); /* k % 256 == 0, 292 B blocks */

/* ---- integer block dots ----
 * number of int32 outputs per row pair: Q4_0/Q8_0 -> k/32 (one isum per block);
 * Q4_K -> 2*k/256 (S1 = sum_j sc_j*isum_j, S2 = sum_j m_j*(bsum_2j + bsum_2j+1));
 * Q6_K -> k/256 (S = sum_s sc_s*isum_s). */
int64_t or_isums_per_row(int wtype, int64_t k);
int or_block_isums(int wtype, const void* wrow, const void* arow, int64_t k, int32_t* out);

/* ---- FrozenMatmul (src/frozen.rs:14-25, src/rie.rs:74-124) ---- */
/* y[t x n] = x[t x k] . W^T   (y overwritten) */
int or_frozen_forward(int wtype, const void* w, int64_t n, int64_t k, const float* x, int64_t t, float* y,
                      int nthreads);
/* same operands, f64 accumulation of the f32-exact block terms (pins the f32 epilogue) */
int or_frozen_forward_f64(int wtype, const void* w, int64_t n, int64_t k, const float* x, int64_t t,
                          double* y);
/* dx[t x k] += dy[t x n] . W */
int or_frozen_backward_input(int wtype, const void* w, int64_t n, int64_t k, const float* dy, int64_t t,
                             float* dx, int nthreads);
int or_frozen_row(int wtype, const void* w, int64_t n, int64_t k, int64_t r, float* out);

/* ---- dense primitives (src/tensor.rs:24-120) ---- */
float or_dot(const float* a, const float* b, int64_t n);
int or_pin_threads(int n); /* timing support: pin an OpenMP team of n to the allowed CPUs */
void or_matmul_nt(const float* a, const float* b, int64_t m, int64_t k, int64_t n, float* out, int nthreads);
void or_matmul_nn(const float* a, const float* b, int64_t m, int64_t k, int64_t n, float* out, int nthreads);
void or_matmul_tn_acc(float* out, const float* a, const float* b, int64_t k, int64_t m, int64_t n,
                      int nthreads);

/* ---- Linear + LoRA (src/linear.rs:73-121) ----
 * A is [r x k], B is [n x r]; scale = alpha / r; lora_enabled 0 bypasses the adapter. */
int or_linear_forward(int wtype, const void* w, int64_t n, int64_t k, const float* bias, int64_t rank,
                      float alpha, const float* A, const float* B, int lora_enabled, const float* x, int64_t t,
                      float* y, int nthreads);
/* dx overwritten (Linear::backward returns a fresh dx); ga [r x k] and gb [n x r] accumulate */
int or_linear_backward(int wtype, const void* w, int64_t n, int64_t k, int64_t rank, float alpha,
                       const float* A, const float* B, int lora_enabled, const float* x, const float* dy,
                       int64_t t, float* dx, float* ga, float* gb, int nthreads);

/* ---- LM head + cross-entropy: Model::head (src/model.rs:561-609) ----
 * For targets i (positions pos[i] into x [t x d], tokens tok[i] < V), in chunks of `chunk` targets:
 * RMSNorm of the target rows (src/ops.rs:14-36), logits = lm_head.forward, softmax_row with an f64
 * normaliser (src/ops.rs:238-247); logp[i] = logit[tok] - lse; *hits = number of targets whose
 * logit is >= every logit.  With wts: dlogits = wts[i] (softmax - onehot), dns = lm_head
 * backward_input, dx (overwritten, [t x d]) += rmsnorm_backward (src/ops.rs:39-56) at pos[i].
 * Returns -1 on a target out of range (the reference asserts). */
int or_lm_head(int wtype, const void* w, int64_t V, int64_t d, const float* norm, float eps, float off,
               const float* x, int64_t t, const int32_t* pos, const int32_t* tok, const float* wts, int64_t n,
               int64_t chunk, float* logp, int64_t* hits, float* dx, int nthreads);
/* ---- model-level training step (rtq_oracle_model.c) ----
 * src/model.rs:644-687 forward_backward_layout over src/model.rs:165-197 Block,
 * src/attention.rs:162-367 Attention, src/model.rs:113-134 Mlp. */
typedef struct {
  int wtype;
  const void* w; /* frozen weight (GGUF blocks, or f32 for OR_F32) */
  int64_t out, in;
  const float* bias; /* [out] or NULL */
  int64_t rank;      /* 0: no adapter */
  float alpha;
  const float* A; /* [rank x in] */
  const float* B; /* [out x rank] */
  float* ga;      /* accumulated gradients, [rank x in] / [out x rank] */
  float* gb;
} or_linear;

typedef struct {
  const float *attn_norm, *ffn_norm; /* [d] */
  const float *q_norm, *k_norm;      /* [head_dim], or NULL without QK-norm */
  or_linear q, k, v, o, gate, up, down;
} or_layer;

typedef struct {
  int n_layer;
  int64_t d, n_head, n_kv, hd, rot, n_ff;
  float eps, off, theta, freq_scale;
  int neox, kv_f16;
  or_linear embed, lm_head; /* the same weight twice when tied; no adapters on either */
  const float* out_norm;
  const or_layer* layers;
  const float* rope_factors; /* per-frequency divisors (rope_freqs.weight), or NULL */
  int64_t n_factors;
} or_model;

/* round_f16 (src/attention.rs:34-51) */
float or_round_f16(float x);
/* Rope tables for positions 0..t-1 (src/ops.rs:141-167): cos / sin [t x rot/2] */
void or_rope_table(int64_t t, int64_t rot, float theta, float freq_scale, float* cos_, float* sin_);
/* Rope::at_positions (src/ops.rs:141-167): tables for tokens at positions[p] (NULL: p), with the
 * inverse frequency of pair i divided by factors[i] where i < n_factors and factors[i] != 0 */
void or_rope_table_at(const int32_t* positions, int64_t t, int64_t rot, float theta, float freq_scale,
                      const float* factors, int64_t n_factors, float* cos_, float* sin_);
/* Rope::allowed (src/ops.rs:160-167): causal, and within the segment layout (seg NULL: plain) */
int or_allowed(const int32_t* seg, int64_t i, int64_t j);

/* ---- the block's operations (teacher-forced parity of a device step, op by op) ---- */
/* rmsnorm_ordered (src/ops.rs:14-36): y, inv [rows]; fused selects x * (inv * w) over (x * inv) * w */
void or_rmsnorm(const float* x, const float* w, int64_t rows, int64_t d, float eps, float off, int fused, float* y,
                float* inv);
/* rmsnorm_backward (src/ops.rs:39-56): dx overwritten */
void or_rmsnorm_backward(const float* x, const float* w, const float* inv, const float* dy, int64_t rows, int64_t d,
                         float off, float* dx);
/* Attention::forward from the raw projections to the rotated heads (src/attention.rs:169-185):
 * QK-norm (q_norm / k_norm may be NULL), RoPE, f16 rounding of k and v when m->kv_f16.
 * q_raw [t x nh x hd], k_raw / v_raw [t x nkv x hd]; q_inv [t nh], k_inv [t nkv] (unused without norms) */
void or_qk_prep(const or_model* m, const float* q_norm, const float* k_norm, const float* cos_, const float* sin_,
                const float* q_raw, const float* k_raw, const float* v_raw, int64_t t, float* q, float* k, float* v,
                float* q_inv, float* k_inv);
/* the backward of or_qk_prep for q and k (src/attention.rs:322-333): inverse RoPE, then the QK-norm
 * backward; dq / dk are not modified */
void or_qk_backward(const or_model* m, const float* q_norm, const float* k_norm, const float* cos_, const float* sin_,
                    const float* q_raw, const float* k_raw, const float* q_inv, const float* k_inv, const float* dq,
                    const float* dk, int64_t t, float* dq_raw, float* dk_raw);
/* causal GQA attention over the allowed pairs (src/attention.rs:187-235): probs [nh x t x t] (zero
 * where not allowed), o [t x nh x hd] */
void or_attention_forward(const or_model* m, const float* q, const float* k, const float* v, int64_t t,
                          const int32_t* seg, float* probs, float* o, int nthreads);
/* its backward (src/attention.rs:262-320): dq [t x nh x hd], dk / dv [t x nkv x hd], overwritten */
void or_attention_backward(const or_model* m, const float* q, const float* k, const float* v, const float* probs,
                           const float* d_o, int64_t t, const int32_t* seg, float* dq, float* dk, float* dv,
                           int nthreads);
/* SwiGLU (src/model.rs:114-119, :123-128): hm = silu(g) u; dg = dhm u silu'(g), du = dhm silu(g) */
void or_swiglu(const float* g, const float* u, int64_t n, float* hm);
void or_swiglu_backward(const float* g, const float* u, const float* dhm, int64_t n, float* dg, float* du);

/* Model::forward_backward (src/model.rs:615-687) on one sequence: logp[n] per target; with wts,
 * the adapters' ga / gb accumulate dL/dA, dL/dB of L = -sum wts[i] logp[i].  Returns -1 on bad
 * shapes or tokens. */
int or_model_forward_backward(const or_model* m, const int32_t* tokens, int64_t t, const int32_t* pos,
                              const int32_t* tok, const float* wts, int64_t n, float* logp, int64_t* hits,
                              int nthreads);
/* forward_backward_layout (src/model.rs:644-687) with a packed layout (Model::forward_backward_packed,
 * :634-642): positions [t] of each token (RoPE) and segments [t] (may-attend rule); either NULL
 * for the plain sequence. */
int or_model_forward_backward_layout(const or_model* m, const int32_t* tokens, int64_t t, const int32_t* positions,
                                     const int32_t* segments, const int32_t* pos, const int32_t* tok,
                                     const float* wts, int64_t n, float* logp, int64_t* hits, int nthreads);
#ifdef __cplusplus
}
#endif
#endif
