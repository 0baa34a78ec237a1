/*
 * rtq_oracle_model.c — CPU restatement of Rust_Trainer's model-level training step over the
 * frozen quantised linears (TEST INFRASTRUCTURE ONLY; see rtq_oracle.h).
 *
 * Restated (files under the reference repository):
 *   src/model.rs:644-687    forward_backward_layout (embed, blocks with checkpointing, head, reverse)
 *   src/model.rs:234-290    Packed / pack (token positions and segments of a shared-prefix batch)
 *   src/model.rs:165-197    Block::forward / backward (pre-norm residual block)
 *   src/model.rs:113-134    Mlp (SwiGLU) forward / backward
 *   src/attention.rs:162-367 Attention forward / backward (QK-norm, RoPE, f16 K/V, causal GQA)
 *   src/attention.rs:34-51  round_f16
 *   src/ops.rs:14-56        rmsnorm_ordered / rmsnorm_backward
 *   src/ops.rs:118-184      Rope (tables in f32 at given positions, per-frequency factors, NEOX / normal
 *                           pairs, inverse = transpose, the segment may-attend rule)
 *   src/tensor.rs:123-143   sigmoid, silu, silu_grad
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "rtq_oracle.h"

/* round_f16 (src/attention.rs:34-51): nearest f16 value, ties to even, as f32 */
float or_round_f16(float x) {
  uint32_t b;
  memcpy(&b, &x, 4);
  const uint32_t sign = b & 0x80000000u, abs_ = b & 0x7fffffffu;
  if (abs_ >= 0x7f800000u) return x;
  const int e = (int)(abs_ >> 23) - 127;
  if (e > 15) {
    const uint32_t r = sign | 0x7f800000u;
    float f;
    memcpy(&f, &r, 4);
    return f;
  }
  const int q_exp = e < -14 ? -24 : e - 10;
  const uint32_t qb = (uint32_t)(q_exp + 127) << 23;
  float q, v;
  memcpy(&q, &qb, 4);
  memcpy(&v, &abs_, 4);
  const float r = rintf(v / q) * q; /* rintf: ties to even in the default rounding mode */
  uint32_t rb;
  memcpy(&rb, &r, 4);
  rb |= sign;
  float out;
  memcpy(&out, &rb, 4);
  return out;
}

/* Rope::at_positions (src/ops.rs:141-167): inv_freq in f32 (divided by a non-zero factor),
 * (pos * f).sin_cos() */
void or_rope_table_at(const int32_t* positions, int64_t t, int64_t rot, float theta, float freq_scale,
                      const float* factors, int64_t n_factors, float* cos_, float* sin_) {
  const int64_t half = rot / 2;
  for (int64_t i = 0; i < half; i++) {
    float f = powf(theta, -2.0f * (float)i / (float)rot) * freq_scale;
    if (factors && i < n_factors && factors[i] != 0.0f) f /= factors[i];
    for (int64_t p = 0; p < t; p++) {
      const float a = (float)(positions ? positions[p] : p) * f;
      cos_[p * half + i] = cosf(a);
      sin_[p * half + i] = sinf(a);
    }
  }
}

void or_rope_table(int64_t t, int64_t rot, float theta, float freq_scale, float* cos_, float* sin_) {
  or_rope_table_at(NULL, t, rot, theta, freq_scale, NULL, 0, cos_, sin_);
}

/* Rope::allowed (src/ops.rs:160-167) */
int or_allowed(const int32_t* seg, int64_t i, int64_t j) {
  return j <= i && (!seg || seg[j] == 0 || seg[j] == seg[i]);
}

/* Rope::apply (src/ops.rs:178-196) on x [t x heads x hd] */
static void rope_apply(const float* cos_, const float* sin_, int64_t rot, int neox, float* x, int64_t t, int64_t heads,
                       int64_t hd, int inverse) {
  const int64_t half = rot / 2;
  const float sgn = inverse ? -1.0f : 1.0f;
  for (int64_t p = 0; p < t; p++)
    for (int64_t h = 0; h < heads; h++) {
      const int64_t base = (p * heads + h) * hd;
      for (int64_t i = 0; i < half; i++) {
        const float c = cos_[p * half + i], s = sgn * sin_[p * half + i];
        const int64_t a = neox ? base + i : base + 2 * i, b = neox ? base + i + half : base + 2 * i + 1;
        const float x1 = x[a], x2 = x[b];
        x[a] = x1 * c - x2 * s;
        x[b] = x2 * c + x1 * s;
      }
    }
}

/* rmsnorm_ordered (src/ops.rs:14-36) */
void or_rmsnorm(const float* x, const float* w, int64_t rows, int64_t d, float eps, float off, int fused, float* y,
                float* inv) {
  for (int64_t r = 0; r < rows; r++) {
    const float* xr = x + r * d;
    const float ms = or_dot(xr, xr, d) / (float)d;
    const float ir = 1.0f / sqrtf(ms + eps);
    inv[r] = ir;
    for (int64_t i = 0; i < d; i++) y[r * d + i] = fused ? xr[i] * (ir * (w[i] + off)) : xr[i] * ir * (w[i] + off);
  }
}

/* rmsnorm_backward (src/ops.rs:39-56) */
void or_rmsnorm_backward(const float* x, const float* w, const float* inv, const float* dy, int64_t rows, int64_t d,
                         float off, float* dx) {
  float* g = (float*)malloc((size_t)d * 4);
  for (int64_t r = 0; r < rows; r++) {
    const float* xr = x + r * d;
    const float* dyr = dy + r * d;
    for (int64_t i = 0; i < d; i++) g[i] = dyr[i] * (w[i] + off);
    const float ir = inv[r];
    const float c = or_dot(g, xr, d) * ir * ir * ir / (float)d;
    for (int64_t i = 0; i < d; i++) dx[r * d + i] = g[i] * ir - xr[i] * c;
  }
  free(g);
}

static float sigmoidf_(float x) {
  if (x >= 0.0f) return 1.0f / (1.0f + expf(-x));
  const float e = expf(x);
  return e / (1.0f + e);
}
static float siluf_(float x) { return x / (1.0f + expf(-x)); }
static float silu_gradf_(float x) {
  const float s = sigmoidf_(x);
  return s * (1.0f + x * (1.0f - s));
}

/* Mlp::forward's activation (src/model.rs:114-119, src/tensor.rs:123-143) */
void or_swiglu(const float* g, const float* u, int64_t n, float* hm) {
  for (int64_t i = 0; i < n; i++) hm[i] = siluf_(g[i]) * u[i];
}

/* Mlp::backward's activation gradient (src/model.rs:123-128) */
void or_swiglu_backward(const float* g, const float* u, const float* dhm, int64_t n, float* dg, float* du) {
  for (int64_t i = 0; i < n; i++) {
    dg[i] = dhm[i] * u[i] * silu_gradf_(g[i]);
    du[i] = dhm[i] * siluf_(g[i]);
  }
}

/* QK-norm, RoPE and f16 K / V (src/attention.rs:169-185) */
void or_qk_prep(const or_model* m, const float* q_norm, const float* k_norm, const float* cos_, const float* sin_,
                const float* q_raw, const float* k_raw, const float* v_raw, int64_t t, float* q, float* k, float* v,
                float* q_inv, float* k_inv) {
  const int64_t nh = m->n_head, nkv = m->n_kv, hd = m->hd, qd = nh * hd, kd = nkv * hd;
  if (q_norm) or_rmsnorm(q_raw, q_norm, t * nh, hd, m->eps, m->off, 1, q, q_inv);
  else memcpy(q, q_raw, (size_t)(t * qd) * 4);
  if (k_norm) or_rmsnorm(k_raw, k_norm, t * nkv, hd, m->eps, m->off, 1, k, k_inv);
  else memcpy(k, k_raw, (size_t)(t * kd) * 4);
  rope_apply(cos_, sin_, m->rot, m->neox, q, t, nh, hd, 0);
  rope_apply(cos_, sin_, m->rot, m->neox, k, t, nkv, hd, 0);
  for (int64_t i = 0; i < t * kd; i++) {
    if (m->kv_f16) k[i] = or_round_f16(k[i]);
    v[i] = m->kv_f16 ? or_round_f16(v_raw[i]) : v_raw[i];
  }
}

/* inverse RoPE, then the QK-norm backward (src/attention.rs:322-333) */
void or_qk_backward(const or_model* m, const float* q_norm, const float* k_norm, const float* cos_, const float* sin_,
                    const float* q_raw, const float* k_raw, const float* q_inv, const float* k_inv, const float* dq,
                    const float* dk, int64_t t, float* dq_raw, float* dk_raw) {
  const int64_t nh = m->n_head, nkv = m->n_kv, hd = m->hd, qd = nh * hd, kd = nkv * hd;
  float* rq = (float*)malloc((size_t)(t * qd) * 4);
  float* rk = (float*)malloc((size_t)(t * kd) * 4);
  memcpy(rq, dq, (size_t)(t * qd) * 4);
  memcpy(rk, dk, (size_t)(t * kd) * 4);
  rope_apply(cos_, sin_, m->rot, m->neox, rq, t, nh, hd, 1);
  rope_apply(cos_, sin_, m->rot, m->neox, rk, t, nkv, hd, 1);
  if (q_norm) or_rmsnorm_backward(q_raw, q_norm, q_inv, rq, t * nh, hd, m->off, dq_raw);
  else memcpy(dq_raw, rq, (size_t)(t * qd) * 4);
  if (k_norm) or_rmsnorm_backward(k_raw, k_norm, k_inv, rk, t * nkv, hd, m->off, dk_raw);
  else memcpy(dk_raw, rk, (size_t)(t * kd) * 4);
  free(rq);
  free(rk);
}

/* per-head attention over the allowed pairs (src/attention.rs:187-235): q scaled first, then dotted
 * with k; max, exp(s - max) and their sum in j order; p = e * (1 / sum); o += p v in j order */
void or_attention_forward(const or_model* m, const float* q, const float* k, const float* v, int64_t t,
                          const int32_t* seg, float* probs, float* o, int nt) {
  const int64_t nh = m->n_head, nkv = m->n_kv, hd = m->hd, grp = nh / nkv;
  const float scale = 1.0f / sqrtf((float)hd);
  memset(probs, 0, (size_t)(nh * t * t) * 4);
  memset(o, 0, (size_t)(t * nh * hd) * 4);
#pragma omp parallel for num_threads(nt > 0 ? nt : 1) schedule(static)
  for (int64_t hh = 0; hh < nh; hh++) {
    const int64_t gg = hh / grp;
    float* qs = (float*)malloc((size_t)hd * 4);
    for (int64_t i = 0; i < t; i++) {
      for (int64_t e = 0; e < hd; e++) qs[e] = q[(i * nh + hh) * hd + e] * scale;
      float* row = probs + (hh * t + i) * t;
      float mx = -INFINITY;
      for (int64_t j = 0; j <= i; j++) {
        if (!or_allowed(seg, i, j)) continue;
        row[j] = or_dot(qs, k + (j * nkv + gg) * hd, hd);
        mx = fmaxf(mx, row[j]);
      }
      float s = 0.0f;
      for (int64_t j = 0; j <= i; j++) {
        if (!or_allowed(seg, i, j)) continue;
        row[j] = expf(row[j] - mx);
        s += row[j];
      }
      const float inv = 1.0f / s;
      float* oi = o + (i * nh + hh) * hd;
      for (int64_t j = 0; j <= i; j++) {
        if (!or_allowed(seg, i, j)) continue;
        row[j] *= inv;
        const float* vj = v + (j * nkv + gg) * hd;
        for (int64_t e = 0; e < hd; e++) oi[e] += row[j] * vj[e];
      }
    }
    free(qs);
  }
}

/* its backward (src/attention.rs:262-320): per head dq, dk, dv; dk / dv summed over the group's
 * heads in head order */
void or_attention_backward(const or_model* m, const float* q, const float* k, const float* v, const float* probs,
                           const float* d_o, int64_t t, const int32_t* seg, float* dq, float* dk, float* dv, int nt) {
  const int64_t nh = m->n_head, nkv = m->n_kv, hd = m->hd, grp = nh / nkv;
  const float scale = 1.0f / sqrtf((float)hd);
  float* dkh_all = (float*)calloc((size_t)(nh * t * hd), 4);
  float* dvh_all = (float*)calloc((size_t)(nh * t * hd), 4);
#pragma omp parallel for num_threads(nt > 0 ? nt : 1) schedule(static)
  for (int64_t hh = 0; hh < nh; hh++) {
    const int64_t gg = hh / grp;
    const float* p = probs + hh * t * t;
    float* dqh = (float*)calloc((size_t)(t * hd), 4);
    float* dkh = dkh_all + hh * t * hd;
    float* dvh = dvh_all + hh * t * hd;
    float* dp = (float*)calloc((size_t)t, 4);
    for (int64_t i = 0; i < t; i++) {
      const float* doi = d_o + (i * nh + hh) * hd;
      float sum = 0.0f;
      for (int64_t j = 0; j <= i; j++) {
        if (!or_allowed(seg, i, j)) continue;
        const float* vj = v + (j * nkv + gg) * hd;
        dp[j] = or_dot(doi, vj, hd);
        sum += p[i * t + j] * dp[j];
        const float pij = p[i * t + j];
        for (int64_t e = 0; e < hd; e++) dvh[j * hd + e] += pij * doi[e];
      }
      const float* qi = q + (i * nh + hh) * hd;
      for (int64_t j = 0; j <= i; j++) {
        if (!or_allowed(seg, i, j)) continue;
        const float ds = p[i * t + j] * (dp[j] - sum) * scale;
        if (ds == 0.0f) continue;
        const float* kj = k + (j * nkv + gg) * hd;
        for (int64_t e = 0; e < hd; e++) dqh[i * hd + e] += ds * kj[e];
        for (int64_t e = 0; e < hd; e++) dkh[j * hd + e] += ds * qi[e];
      }
    }
    for (int64_t i = 0; i < t; i++) memcpy(dq + (i * nh + hh) * hd, dqh + i * hd, (size_t)hd * 4);
    free(dqh);
    free(dp);
  }
  memset(dk, 0, (size_t)(t * nkv * hd) * 4);
  memset(dv, 0, (size_t)(t * nkv * hd) * 4);
  for (int64_t hh = 0; hh < nh; hh++) /* per-head dk / dv summed in head order (src/attention.rs:310-319) */
    for (int64_t i = 0; i < t; i++)
      for (int64_t e = 0; e < hd; e++) {
        dk[(i * nkv + hh / grp) * hd + e] += dkh_all[(hh * t + i) * hd + e];
        dv[(i * nkv + hh / grp) * hd + e] += dvh_all[(hh * t + i) * hd + e];
      }
  free(dkh_all);
  free(dvh_all);
}

static int lin_fwd(const or_linear* l, const float* x, int64_t t, float* y, int nt) {
  return or_linear_forward(l->wtype, l->w, l->out, l->in, l->bias, l->rank, l->alpha, l->A, l->B, l->rank > 0, x, t,
                           y, nt);
}
static int lin_bwd(const or_linear* l, const float* x, const float* dy, int64_t t, float* dx, int nt) {
  return or_linear_backward(l->wtype, l->w, l->out, l->in, l->rank, l->alpha, l->A, l->B, l->rank > 0, x, dy, t, dx,
                            l->ga, l->gb, nt);
}

#define FREE_ALL(...)                                         \
  do {                                                        \
    void* ps_[] = {__VA_ARGS__};                              \
    for (size_t i_ = 0; i_ < sizeof ps_ / sizeof *ps_; i_++) free(ps_[i_]); \
  } while (0)

/* one block: forward (y) and, with dy, backward (dx); dx may alias nothing */
static int block(const or_model* m, const or_layer* L, const float* cos_, const float* sin_, const int32_t* seg,
                 const float* x, int64_t t, float* y, const float* dy, float* dx, int nt) {
  const int64_t d = m->d, nh = m->n_head, nkv = m->n_kv, hd = m->hd, ff = m->n_ff;
  const int64_t qd = nh * hd, kd = nkv * hd;
  float* inv1 = (float*)malloc((size_t)t * 4);
  float* n1 = (float*)malloc((size_t)(t * d) * 4);
  float* q_raw = (float*)malloc((size_t)(t * qd) * 4);
  float* k_raw = (float*)malloc((size_t)(t * kd) * 4);
  float* v_raw = (float*)malloc((size_t)(t * kd) * 4);
  float* v = (float*)malloc((size_t)(t * kd) * 4);
  float* q = (float*)malloc((size_t)(t * qd) * 4);
  float* k = (float*)malloc((size_t)(t * kd) * 4);
  float* q_inv = (float*)malloc((size_t)(t * nh) * 4);
  float* k_inv = (float*)malloc((size_t)(t * nkv) * 4);
  float* probs = (float*)malloc((size_t)(nh * t * t) * 4);
  float* o = (float*)malloc((size_t)(t * qd) * 4);
  float* mo = (float*)malloc((size_t)(t * d) * 4);
  float* h = (float*)malloc((size_t)(t * d) * 4);
  float* inv2 = (float*)malloc((size_t)t * 4);
  float* n2 = (float*)malloc((size_t)(t * d) * 4);
  float* g = (float*)malloc((size_t)(t * ff) * 4);
  float* u = (float*)malloc((size_t)(t * ff) * 4);
  float* hm = (float*)malloc((size_t)(t * ff) * 4);
  float* f = (float*)malloc((size_t)(t * d) * 4);
  int rc = 0;
  /* ---- forward (src/model.rs:166-180, src/attention.rs:162-240, src/model.rs:114-119) */
  or_rmsnorm(x, L->attn_norm, t, d, m->eps, m->off, 0, n1, inv1);
  if ((rc = lin_fwd(&L->q, n1, t, q_raw, nt)) || (rc = lin_fwd(&L->k, n1, t, k_raw, nt)) ||
      (rc = lin_fwd(&L->v, n1, t, v_raw, nt)))
    goto out;
  or_qk_prep(m, L->q_norm, L->k_norm, cos_, sin_, q_raw, k_raw, v_raw, t, q, k, v, q_inv, k_inv);
  or_attention_forward(m, q, k, v, t, seg, probs, o, nt);
  if ((rc = lin_fwd(&L->o, o, t, mo, nt))) goto out;
  for (int64_t i = 0; i < t * d; i++) h[i] = x[i] + mo[i];
  or_rmsnorm(h, L->ffn_norm, t, d, m->eps, m->off, 0, n2, inv2);
  if ((rc = lin_fwd(&L->gate, n2, t, g, nt)) || (rc = lin_fwd(&L->up, n2, t, u, nt))) goto out;
  or_swiglu(g, u, t * ff, hm);
  if ((rc = lin_fwd(&L->down, hm, t, f, nt))) goto out;
  if (y)
    for (int64_t i = 0; i < t * d; i++) y[i] = h[i] + f[i];
  if (!dy) goto out;
  /* ---- backward (src/model.rs:183-194) */
  {
    float* dhm = (float*)malloc((size_t)(t * ff) * 4);
    float* dg = (float*)malloc((size_t)(t * ff) * 4);
    float* du = (float*)malloc((size_t)(t * ff) * 4);
    float* dn2 = (float*)malloc((size_t)(t * d) * 4);
    float* dxu = (float*)malloc((size_t)(t * d) * 4);
    float* dh = (float*)malloc((size_t)(t * d) * 4);
    float* d_o = (float*)malloc((size_t)(t * qd) * 4);
    float* dq = (float*)malloc((size_t)(t * qd) * 4);
    float* dk = (float*)malloc((size_t)(t * kd) * 4);
    float* dv = (float*)malloc((size_t)(t * kd) * 4);
    float* dq_raw = (float*)malloc((size_t)(t * qd) * 4);
    float* dk_raw = (float*)malloc((size_t)(t * kd) * 4);
    float* dn1 = (float*)malloc((size_t)(t * d) * 4);
    float* dxk = (float*)malloc((size_t)(t * d) * 4);
    float* dxv = (float*)malloc((size_t)(t * d) * 4);
    /* Mlp::backward (src/model.rs:120-133) */
    if ((rc = lin_bwd(&L->down, hm, dy, t, dhm, nt))) goto bout;
    or_swiglu_backward(g, u, dhm, t * ff, dg, du);
    if ((rc = lin_bwd(&L->gate, n2, dg, t, dn2, nt)) || (rc = lin_bwd(&L->up, n2, du, t, dxu, nt))) goto bout;
    for (int64_t i = 0; i < t * d; i++) dn2[i] += dxu[i];
    or_rmsnorm_backward(h, L->ffn_norm, inv2, dn2, t, d, m->off, dh);
    for (int64_t i = 0; i < t * d; i++) dh[i] = dy[i] + dh[i];
    /* Attention::backward (src/attention.rs:243-355) */
    if ((rc = lin_bwd(&L->o, o, dh, t, d_o, nt))) goto bout;
    or_attention_backward(m, q, k, v, probs, d_o, t, seg, dq, dk, dv, nt);
    or_qk_backward(m, L->q_norm, L->k_norm, cos_, sin_, q_raw, k_raw, q_inv, k_inv, dq, dk, t, dq_raw, dk_raw);
    if ((rc = lin_bwd(&L->q, n1, dq_raw, t, dn1, nt)) || (rc = lin_bwd(&L->k, n1, dk_raw, t, dxk, nt)) ||
        (rc = lin_bwd(&L->v, n1, dv, t, dxv, nt)))
      goto bout;
    for (int64_t i = 0; i < t * d; i++) dn1[i] += dxk[i] + dxv[i];
    or_rmsnorm_backward(x, L->attn_norm, inv1, dn1, t, d, m->off, dx);
    for (int64_t i = 0; i < t * d; i++) dx[i] = dh[i] + dx[i];
  bout:
    FREE_ALL(dhm, dg, du, dn2, dxu, dh, d_o, dq, dk, dv, dq_raw, dk_raw, dn1, dxk, dxv);
  }
out:
  FREE_ALL(inv1, n1, q_raw, k_raw, v_raw, v, q, k, q_inv, k_inv, probs, o, mo, h, inv2, n2, g, u, hm, f);
  return rc;
}

int or_model_forward_backward_layout(const or_model* m, const int32_t* tokens, int64_t t, const int32_t* positions,
                                     const int32_t* segments, const int32_t* pos, const int32_t* tok,
                                     const float* wts, int64_t n, float* logp, int64_t* hits, int nthreads) {
  const int64_t d = m->d;
  if (t <= 0 || m->n_head % m->n_kv || m->rot % 2 || m->rot > m->hd) return -1;
  for (int64_t i = 0; i < t; i++)
    if (tokens[i] < 0 || tokens[i] >= m->embed.out) return -1; /* src/model.rs:450 */
  if (positions)
    for (int64_t i = 0; i < t; i++)
      if (positions[i] < 0) return -1;
  float* cos_ = (float*)malloc((size_t)(t * (m->rot / 2) + 1) * 4);
  float* sin_ = (float*)malloc((size_t)(t * (m->rot / 2) + 1) * 4);
  /* Model::rope_for (src/model.rs:461-481) */
  or_rope_table_at(positions, t, m->rot, m->theta, m->freq_scale, m->rope_factors, m->n_factors, cos_, sin_);
  float* inputs = (float*)malloc((size_t)(m->n_layer + 1) * (size_t)(t * d) * 4); /* checkpoints */
  float* dx = (float*)malloc((size_t)(t * d) * 4);
  float* dx2 = (float*)malloc((size_t)(t * d) * 4);
  int rc = 0;
  for (int64_t i = 0; i < t && !rc; i++) /* embed_tokens (src/model.rs:446-454) */
    rc = or_frozen_row(m->embed.wtype, m->embed.w, m->embed.out, m->embed.in, tokens[i], inputs + i * d);
  for (int l = 0; l < m->n_layer && !rc; l++)
    rc = block(m, &m->layers[l], cos_, sin_, segments, inputs + (size_t)l * (size_t)(t * d), t,
               inputs + (size_t)(l + 1) * (size_t)(t * d), NULL, NULL, nthreads);
  if (!rc)
    rc = or_lm_head(m->lm_head.wtype, m->lm_head.w, m->lm_head.out, d, m->out_norm, m->eps, m->off,
                    inputs + (size_t)m->n_layer * (size_t)(t * d), t, pos, tok, wts, n, 64, logp, hits, dx, nthreads);
  for (int l = m->n_layer - 1; l >= 0 && !rc && wts; l--) { /* recompute each block, then backward */
    rc = block(m, &m->layers[l], cos_, sin_, segments, inputs + (size_t)l * (size_t)(t * d), t, NULL, dx, dx2,
               nthreads);
    float* s = dx;
    dx = dx2;
    dx2 = s;
  }
  free(cos_);
  free(sin_);
  free(inputs);
  free(dx);
  free(dx2);
  return rc;
}

int or_model_forward_backward(const or_model* m, const int32_t* tokens, int64_t t, const int32_t* pos,
                              const int32_t* tok, const float* wts, int64_t n, float* logp, int64_t* hits,
                              int nthreads) {
  return or_model_forward_backward_layout(m, tokens, t, NULL, NULL, pos, tok, wts, n, logp, hits, nthreads);
}
