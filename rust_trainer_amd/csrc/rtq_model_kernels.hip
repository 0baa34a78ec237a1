// rtq_model_kernels.hip — the decoder block around the frozen linears, for the device-resident
// training step (rtq_model_* in include/rtq.h).  Included by rtq_kernels.hip (one code object).
//
// Reference operations restated (files under the reference repository):
//   rmsnorm_ordered / rmsnorm_backward     src/ops.rs:14-56
//   Rope::apply (NEOX / normal pairs)       src/ops.rs:178-196
//   round_f16                               src/attention.rs:34-51
//   Attention forward / backward            src/attention.rs:162-367 (causal GQA, probabilities kept)
//   Mlp (SwiGLU), sigmoid / silu / grad     src/model.rs:113-134, src/tensor.rs:123-143
// Arithmetic follows the reference's f32 operation order element by element; reductions (norm
// sums, softmax sums, dot products) are tree-ordered.

// ------------------------------------------------------------------ helpers
__device__ __forceinline__ float m_round_f16(float x) {
  const uint32_t b = __float_as_uint(x);
  const uint32_t sign = b & 0x80000000u, abs_ = b & 0x7fffffffu;
  if (abs_ >= 0x7f800000u) return x;
  const int e = (int)(abs_ >> 23) - 127;
  if (e > 15) return __uint_as_float(sign | 0x7f800000u);
  const int q_exp = e < -14 ? -24 : e - 10;
  const float q = __uint_as_float((uint32_t)(q_exp + 127) << 23);
  const float r = __fmul_rn(rintf(__fdiv_rn(__uint_as_float(abs_), q)), q);
  return __uint_as_float(sign | __float_as_uint(r));
}

__device__ __forceinline__ float m_sigmoid(float x) { return rtq_sigmoid(x); }
__device__ __forceinline__ float m_silu(float x) { return rtq_silu(x); }
__device__ __forceinline__ float m_silu_grad(float x) { return rtq_silu_grad(x); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
  return v;
}

// ------------------------------------------------------------------ RMSNorm
// One workgroup of 256 threads per row; thread i takes columns i, i + 256, ...
// The backward holds rows up to 256 NPT columns in registers, so that all of its loads are issued
// up front (one memory round trip before the row sum; 401 -> 331 us per Qwen3-0.6B-shaped
// 512-token step); longer rows stream twice.  (The same in the forward measured slower: 342 -> 382.)
constexpr int RTQ_NORM_NPT = 16;

// wave-per-row layout: lane l takes the float4 columns 4 l + 256 i (i < d / 256, at most 8)
constexpr int RTQ_NORM_WV = 8;

// grid rows (wave: rows / 4), 256 threads: y = rmsnorm(a (+ b)); with b, h = a + b is written too
extern "C" __global__ __launch_bounds__(256) void rtq_m_rmsnorm(MNormArgs a) {
  if (a.wave) {  // one wave per row: no workgroup barrier, every load issued at once
    const int r = (int)(blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)), lane = threadIdx.x & 63, nv = a.d / 256;
    if (r >= a.rows) return;
    const int64_t ro = (int64_t)r * a.d + 4 * lane;
    f4 xv[RTQ_NORM_WV], wv[RTQ_NORM_WV];
#pragma unroll
    for (int i = 0; i < RTQ_NORM_WV; i++)
      if (i < nv) {
        xv[i] = *reinterpret_cast<const f4*>(a.a + ro + 256 * i);
        wv[i] = *reinterpret_cast<const f4*>(a.w + 4 * lane + 256 * i);
        if (a.b) xv[i] += *reinterpret_cast<const f4*>(a.b + ro + 256 * i);
      }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < RTQ_NORM_WV; i++)
      if (i < nv) {
        if (a.b) *reinterpret_cast<f4*>(a.h + ro + 256 * i) = xv[i];
#pragma unroll
        for (int e = 0; e < 4; e++) s = s + xv[i][e] * xv[i][e];
      }
    s = wave_sum(s);
    const float ir = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(s, (float)a.d) + a.eps));
#pragma unroll
    for (int i = 0; i < RTQ_NORM_WV; i++)
      if (i < nv) {
        f4 y;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const float x = xv[i][e], wo = wv[i][e] + a.off;
          y[e] = a.fused ? x * (ir * wo) : (x * ir) * wo;
        }
        *reinterpret_cast<f4*>(a.y + ro + 256 * i) = y;
      }
    if (lane == 0) a.inv[r] = ir;
    return;
  }
  __shared__ float red[4];
  const int r = blockIdx.x, tid = threadIdx.x;
  const float* ar = a.a + (int64_t)r * a.d;
  const float* br = a.b ? a.b + (int64_t)r * a.d : nullptr;
  float* hr = a.b ? a.h + (int64_t)r * a.d : nullptr;
  float* yr = a.y + (int64_t)r * a.d;
  float s = 0.0f;
  for (int k = tid; k < a.d; k += 256) {
    float x = ar[k];
    if (br) {
      x = x + br[k];
      hr[k] = x;
    }
    s = s + x * x;
  }
  s = block_sum256(s, red);
  const float ir = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(s, (float)a.d) + a.eps));
  const float* xr = br ? hr : ar;
  for (int k = tid; k < a.d; k += 256) {
    const float x = xr[k], wo = a.w[k] + a.off;
    yr[k] = a.fused ? x * (ir * wo) : (x * ir) * wo;
  }
  if (tid == 0) a.inv[r] = ir;
}

// grid rows (wave: rows / 4), 256 threads: out = (res +) rmsnorm_backward(x, w, inv, dy)
extern "C" __global__ __launch_bounds__(256) void rtq_m_rmsnorm_bwd(MNormBwdArgs a) {
  if (a.wave) {  // one wave per row, as the forward
    const int r = (int)(blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)), lane = threadIdx.x & 63, nv = a.d / 256;
    if (r >= a.rows) return;
    const int64_t ro = (int64_t)r * a.d + 4 * lane;
    const float ir = a.inv[r];
    f4 xv[RTQ_NORM_WV], gv[RTQ_NORM_WV], rv[RTQ_NORM_WV];
#pragma unroll
    for (int i = 0; i < RTQ_NORM_WV; i++)
      if (i < nv) {
        xv[i] = *reinterpret_cast<const f4*>(a.x + ro + 256 * i);
        const f4 dv = *reinterpret_cast<const f4*>(a.dy + ro + 256 * i);
        const f4 wv = *reinterpret_cast<const f4*>(a.w + 4 * lane + 256 * i);
#pragma unroll
        for (int e = 0; e < 4; e++) gv[i][e] = dv[e] * (wv[e] + a.off);
        if (a.res) rv[i] = *reinterpret_cast<const f4*>(a.res + ro + 256 * i);
      }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < RTQ_NORM_WV; i++)
      if (i < nv)
#pragma unroll
        for (int e = 0; e < 4; e++) s = s + gv[i][e] * xv[i][e];
    s = wave_sum(s);
    const float c = __fdiv_rn(((s * ir) * ir) * ir, (float)a.d);
#pragma unroll
    for (int i = 0; i < RTQ_NORM_WV; i++)
      if (i < nv) {
        f4 o;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const float v = gv[i][e] * ir - xv[i][e] * c;
          o[e] = a.res ? rv[i][e] + v : v;
        }
        *reinterpret_cast<f4*>(a.out + ro + 256 * i) = o;
      }
    return;
  }
  __shared__ float red[4];
  const int r = blockIdx.x, tid = threadIdx.x;
  const float* xr = a.x + (int64_t)r * a.d;
  const float* dr = a.dy + (int64_t)r * a.d;
  float* o = a.out + (int64_t)r * a.d;
  const float* rr = a.res ? a.res + (int64_t)r * a.d : nullptr;
  const float ir = a.inv[r];
  if (a.d <= 256 * RTQ_NORM_NPT) {
    float gv[RTQ_NORM_NPT], xv[RTQ_NORM_NPT], rv[RTQ_NORM_NPT];
#pragma unroll
    for (int i = 0; i < RTQ_NORM_NPT; i++) {
      const int k = tid + 256 * i;
      const bool in = k < a.d;
      xv[i] = in ? xr[k] : 0.0f;
      gv[i] = in ? dr[k] * (a.w[k] + a.off) : 0.0f;
      rv[i] = in && rr ? rr[k] : 0.0f;
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < RTQ_NORM_NPT; i++)
      if (tid + 256 * i < a.d) s = s + gv[i] * xv[i];
    s = block_sum256(s, red);
    const float c = __fdiv_rn(((s * ir) * ir) * ir, (float)a.d);
#pragma unroll
    for (int i = 0; i < RTQ_NORM_NPT; i++) {
      const int k = tid + 256 * i;
      const float v = gv[i] * ir - xv[i] * c;
      if (k < a.d) o[k] = rr ? rv[i] + v : v;
    }
    return;
  }
  float s = 0.0f;
  for (int k = tid; k < a.d; k += 256) s = s + (dr[k] * (a.w[k] + a.off)) * xr[k];
  s = block_sum256(s, red);
  const float c = __fdiv_rn(((s * ir) * ir) * ir, (float)a.d);
  for (int k = tid; k < a.d; k += 256) {
    const float g = dr[k] * (a.w[k] + a.off);
    const float v = g * ir - xr[k] * c;
    o[k] = rr ? rr[k] + v : v;
  }
}

// ------------------------------------------------------------------ QK-norm + RoPE + f16 K/V
// One wave per (token, head) row of width hd (hd <= 512): rows [0, t nh) are q, then t nkv k rows,
// then t nkv v rows.  LDS holds the normalised row so the RoPE pairs can be read across lanes.
// rotates the row src into dst (sgn -1: the inverse rotation), rounding to f16 when rnd
__device__ __forceinline__ void m_rope_row(const MQkArgs& a, const float* src, float* dst, int p, float sgn, bool rnd) {
  const int half = a.rot / 2, lane = threadIdx.x & 63;
  const float* cr = a.cos_ + (int64_t)p * half;
  const float* sr = a.sin_ + (int64_t)p * half;
  for (int i = lane; i < half; i += 64) {
    const float c = cr[i], s = sgn * sr[i];
    const int ia = a.neox ? i : 2 * i, ib = a.neox ? i + half : 2 * i + 1;
    const float x1 = src[ia], x2 = src[ib];
    const float y1 = x1 * c - x2 * s, y2 = x2 * c + x1 * s;
    dst[ia] = rnd ? m_round_f16(y1) : y1;
    dst[ib] = rnd ? m_round_f16(y2) : y2;
  }
  for (int e = a.rot + lane; e < a.hd; e += 64) dst[e] = rnd ? m_round_f16(src[e]) : src[e];
}

// half-wave rows (hd = rot = 128): lane l (of 32) holds elements 4 l .. 4 l + 3.  RoPE of those four
// (sgn -1: the inverse rotation); NEOX pairs (i, i + 64) sit in lanes l and l ^ 16 of the half-wave
__device__ __forceinline__ f4 m_rope_h(const MQkArgs& a, f4 y, int p, float sgn) {
  const int l = threadIdx.x & 31;
  f4 out;
  if (a.neox) {
    const int i0 = 4 * (l & 15);
    const f4 c = *reinterpret_cast<const f4*>(a.cos_ + (int64_t)p * 64 + i0);
    const f4 sn = *reinterpret_cast<const f4*>(a.sin_ + (int64_t)p * 64 + i0);
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const float other = __shfl_xor(y[e], 16), s = sgn * sn[e];
      out[e] = l < 16 ? y[e] * c[e] - other * s : y[e] * c[e] + other * s;  // x1 c - x2 s | x2 c + x1 s
    }
  } else {
    const float2 c = *reinterpret_cast<const float2*>(a.cos_ + (int64_t)p * 64 + 2 * l);
    const float2 sn = *reinterpret_cast<const float2*>(a.sin_ + (int64_t)p * 64 + 2 * l);
    const float s0 = sgn * sn.x, s1 = sgn * sn.y;
    out[0] = y[0] * c.x - y[1] * s0;
    out[1] = y[1] * c.x + y[0] * s0;
    out[2] = y[2] * c.y - y[3] * s1;
    out[3] = y[3] * c.y + y[2] * s1;
  }
  return out;
}
__device__ __forceinline__ float half_sum(float v) {
#pragma unroll
  for (int m = 1; m <= 16; m <<= 1) v += __shfl_xor(v, m);
  return v;
}

extern "C" __global__ __launch_bounds__(256) void rtq_m_qk_prep(MQkArgs a) {
  if (a.half) {  // half-wave per row, every load issued at once
    const int l = threadIdx.x & 31;
    const int64_t row = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
    const int64_t nq = (int64_t)a.t * a.nh, nk = (int64_t)a.t * a.nkv;
    if (row >= nq + 2 * nk) return;  // the whole half-wave
    if (row >= nq + nk) {  // v: f16 rounding only
      const int64_t rv = row - nq - nk;
      f4 x = *reinterpret_cast<const f4*>(a.v_raw + (rv / a.nkv) * a.ldv + (rv % a.nkv) * 128 + 4 * l);
      if (a.kv_f16)
#pragma unroll
        for (int e = 0; e < 4; e++) x[e] = m_round_f16(x[e]);
      *reinterpret_cast<f4*>(a.v + rv * 128 + 4 * l) = x;
      return;
    }
    const bool isq = row < nq;
    const int64_t r = isq ? row : row - nq;
    const int heads = isq ? a.nh : a.nkv, p = (int)(r / heads);
    f4 y = *reinterpret_cast<const f4*>((isq ? a.q_raw + p * a.ldq : a.k_raw + p * a.ldk) + (r % heads) * 128 + 4 * l);
    const float* w = isq ? a.q_norm : a.k_norm;
    if (w) {
      const f4 wv = *reinterpret_cast<const f4*>(w + 4 * l);
      float s = 0.0f;
#pragma unroll
      for (int e = 0; e < 4; e++) s = s + y[e] * y[e];
      s = half_sum(s);
      const float ir = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(s, 128.0f) + a.eps));
#pragma unroll
      for (int e = 0; e < 4; e++) y[e] = y[e] * (ir * (wv[e] + a.off));
      if (l == 0) (isq ? a.q_inv : a.k_inv)[r] = ir;
    }
    f4 o = m_rope_h(a, y, p, 1.0f);
    if (!isq && a.kv_f16)
#pragma unroll
      for (int e = 0; e < 4; e++) o[e] = m_round_f16(o[e]);
    *reinterpret_cast<f4*>((isq ? a.q : a.k) + r * 128 + 4 * l) = o;
    return;
  }
  __shared__ float buf[4][512];
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + wv;
  const int64_t nq = (int64_t)a.t * a.nh, nk = (int64_t)a.t * a.nkv;
  if (row >= nq + 2 * nk) return;
  float* sb = buf[wv];
  if (row >= nq + nk) {  // v: f16 rounding only
    const int64_t rv = row - nq - nk, o = rv * a.hd;
    const float* vr = a.v_raw + (rv / a.nkv) * a.ldv + (rv % a.nkv) * a.hd;
    for (int e = lane; e < a.hd; e += 64) a.v[o + e] = a.kv_f16 ? m_round_f16(vr[e]) : vr[e];
    return;
  }
  const bool isq = row < nq;
  const int64_t r = isq ? row : row - nq;
  const int heads = isq ? a.nh : a.nkv;
  const int p = (int)(r / heads);
  const float* x = (isq ? a.q_raw + p * a.ldq : a.k_raw + p * a.ldk) + (r % heads) * a.hd;
  const float* w = isq ? a.q_norm : a.k_norm;
  if (w && a.hd <= 256) {  // the row in registers: its loads issued together
    float xv[4], wv[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int e = min(lane + 64 * u, a.hd - 1);
      xv[u] = x[e];
      wv[u] = w[e];
    }
    float s = 0.0f;
#pragma unroll
    for (int u = 0; u < 4; u++)
      if (lane + 64 * u < a.hd) s = s + xv[u] * xv[u];
    s = wave_sum(s);
    const float ir = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(s, (float)a.hd) + a.eps));
#pragma unroll
    for (int u = 0; u < 4; u++)
      if (lane + 64 * u < a.hd) sb[lane + 64 * u] = xv[u] * (ir * (wv[u] + a.off));
    if (lane == 0) (isq ? a.q_inv : a.k_inv)[r] = ir;
  } else if (w) {
    float s = 0.0f;
    for (int e = lane; e < a.hd; e += 64) s = s + x[e] * x[e];
    s = wave_sum(s);
    const float ir = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(s, (float)a.hd) + a.eps));
    for (int e = lane; e < a.hd; e += 64) sb[e] = x[e] * (ir * (w[e] + a.off));
    if (lane == 0) (isq ? a.q_inv : a.k_inv)[r] = ir;
  } else {
    for (int e = lane; e < a.hd; e += 64) sb[e] = x[e];
  }
  __builtin_amdgcn_wave_barrier();
  m_rope_row(a, sb, (isq ? a.q : a.k) + r * a.hd, p, 1.0f, !isq && a.kv_f16);
}

// backward: dq_raw / dk_raw = rmsnorm_backward(inverse RoPE of dq / dk); rows [0, t nh) q, then k
extern "C" __global__ __launch_bounds__(256) void rtq_m_qk_bwd(MQkArgs a) {
  if (a.half) {  // half-wave per row, as the forward
    const int l = threadIdx.x & 31;
    const int64_t row = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
    const int64_t nq = (int64_t)a.t * a.nh, nk = (int64_t)a.t * a.nkv;
    if (row >= nq + nk) return;
    const bool isq = row < nq;
    const int64_t r = isq ? row : row - nq;
    const int heads = isq ? a.nh : a.nkv, p = (int)(r / heads);
    const int64_t roff = (isq ? p * a.ldq : p * a.ldk) + (r % heads) * 128 + 4 * l;
    const float* w = isq ? a.q_norm : a.k_norm;
    f4 xv = {0.0f, 0.0f, 0.0f, 0.0f}, wv = xv;
    if (w) {
      xv = *reinterpret_cast<const f4*>((isq ? a.q_raw : a.k_raw) + roff);
      wv = *reinterpret_cast<const f4*>(w + 4 * l);
    }
    f4 g;
    const int mi = a.qmi ? (isq ? a.qmi : a.kmi)[(r % heads) * a.nb16 + (p >> 4)] : -1;
    if (mi >= 0) {  // a cut block: its slots in order (dq; dk, and the row's dv written here)
      const MAttnMerge mg = (isq ? a.qmerges : a.kmerges)[mi];
      const float* s0 = (isq ? a.qpart : a.kpart) + (int64_t)mg.s0 * 4096 + (p & 15) * 128 + 4 * l;
      g = f4{0.0f, 0.0f, 0.0f, 0.0f};
      f4 dvs = g;
      for (int k = 0; k < mg.n; k++) {
        g += *reinterpret_cast<const f4*>(s0 + (int64_t)k * 4096);
        if (!isq) dvs += *reinterpret_cast<const f4*>(s0 + (int64_t)k * 4096 + 2048);
      }
      if (!isq) *reinterpret_cast<f4*>(a.dv + p * a.ld_dv + (r % heads) * 128 + 4 * l) = dvs;
    } else {
      g = *reinterpret_cast<const f4*>((isq ? a.dq : a.dk) + r * 128 + 4 * l);
    }
    const f4 sb = m_rope_h(a, g, p, -1.0f);
    float* out = (isq ? a.dq_raw : a.dk_raw) + roff;
    if (!w) {
      *reinterpret_cast<f4*>(out) = sb;
      return;
    }
    const float ir = (isq ? a.q_inv : a.k_inv)[r];
    f4 gv;
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      gv[e] = sb[e] * (wv[e] + a.off);
      s = s + gv[e] * xv[e];
    }
    s = half_sum(s);
    const float c = __fdiv_rn(((s * ir) * ir) * ir, 128.0f);
    f4 o;
#pragma unroll
    for (int e = 0; e < 4; e++) o[e] = gv[e] * ir - xv[e] * c;
    *reinterpret_cast<f4*>(out) = o;
    return;
  }
  __shared__ float buf[4][512];
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + wv;
  const int64_t nq = (int64_t)a.t * a.nh, nk = (int64_t)a.t * a.nkv;
  if (row >= nq + nk) return;
  const bool isq = row < nq;
  const int64_t r = isq ? row : row - nq;
  const int heads = isq ? a.nh : a.nkv;
  const int p = (int)(r / heads);
  float* sb = buf[wv];
  const int64_t roff = (isq ? p * a.ldq : p * a.ldk) + (r % heads) * a.hd;
  float* out = (isq ? a.dq_raw : a.dk_raw) + roff;
  const float* w = isq ? a.q_norm : a.k_norm;
  const float* x = (isq ? a.q_raw : a.k_raw) + roff;
  if (w && a.hd <= 256) {  // the norm's operands loaded before the rotation, all together
    float xv[4], wv[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int e = min(lane + 64 * u, a.hd - 1);
      xv[u] = x[e];
      wv[u] = w[e];
    }
    const float ir = (isq ? a.q_inv : a.k_inv)[r];
    m_rope_row(a, (isq ? a.dq : a.dk) + r * a.hd, sb, p, -1.0f, false);
    __builtin_amdgcn_wave_barrier();
    float gv[4];
    float s = 0.0f;
#pragma unroll
    for (int u = 0; u < 4; u++) {
      gv[u] = lane + 64 * u < a.hd ? sb[lane + 64 * u] * (wv[u] + a.off) : 0.0f;
      if (lane + 64 * u < a.hd) s = s + gv[u] * xv[u];
    }
    s = wave_sum(s);
    const float c = __fdiv_rn(((s * ir) * ir) * ir, (float)a.hd);
#pragma unroll
    for (int u = 0; u < 4; u++)
      if (lane + 64 * u < a.hd) out[lane + 64 * u] = gv[u] * ir - xv[u] * c;
    return;
  }
  m_rope_row(a, (isq ? a.dq : a.dk) + r * a.hd, sb, p, -1.0f, false);
  __builtin_amdgcn_wave_barrier();
  if (!w) {
    for (int e = lane; e < a.hd; e += 64) out[e] = sb[e];
    return;
  }
  const float ir = (isq ? a.q_inv : a.k_inv)[r];
  float s = 0.0f;
  for (int e = lane; e < a.hd; e += 64) s = s + (sb[e] * (w[e] + a.off)) * x[e];
  s = wave_sum(s);
  const float c = __fdiv_rn(((s * ir) * ir) * ir, (float)a.hd);
  for (int e = lane; e < a.hd; e += 64) {
    const float g = sb[e] * (w[e] + a.off);
    out[e] = g * ir - x[e] * c;
  }
}

// ------------------------------------------------------------------ batched f32 GEMM
// C(b) (+)= A(b) B(b) on f32 MFMA (16x16x4: exact f32 products, f32 accumulation), a BM x 64 output
// tile per 256-thread workgroup, k slabs of BK through LDS.  MFMA q of a 16-deep k group takes
// k = 16 kb + 4 g + q in k slot g of A and of B alike.  An operand whose global unit-stride index is
// k (mode 1) sits in LDS as [row][k] and a lane reads its 4 k with one 16-byte read; one whose
// unit-stride index is the row (mode 2) sits as [k][row] and is read by 4 single reads.  Both are
// loaded and stored as 16-byte vectors along the unit-stride index (when the other strides, the
// extent and the base allow); otherwise single floats in the mode-1 arrangement (mode 0).  The next
// slab is loaded into registers while the current one feeds the MFMAs.
// Waves 2 x 2: BM = 64, 32 x 32 each (2 x 2 MFMA tiles); BM = 32, 16 x 32 (1 x 2).
template <int BM>
struct MGemmCfg {
  // 32-row tiles serve the long-K products (O, dV, dQ, dK: K = t): 64-deep slabs; 64-row tiles the
  // K = head_dim ones: 32-deep slabs
  static constexpr int BN = 64, BK = BM == 32 ? 64 : 32;
  static constexpr int NA = BM * BK / 1024, NB = BN * BK / 1024;  // float4 per thread and slab
  static constexpr int TM = BM / 32;                              // 16-row MFMA tiles per wave
};
// LDS floats of an R x BK operand in either layout: [R][BK + 4] or [BK][R + 4]
template <int R, int BK>
constexpr int m_opnd_lds() { return R * (BK + 4) > BK * (R + 4) ? R * (BK + 4) : BK * (R + 4); }

// load mode of an operand whose element (r, k) is P[r * sr + k * sk] (P already offset to its batch)
__device__ __forceinline__ int m_opnd_mode(const float* P, int64_t sr, int64_t sk, int64_t sb, int nrows, int K) {
  const bool al = (reinterpret_cast<uintptr_t>(P) & 15u) == 0 && sb % 4 == 0;
  if (al && sk == 1 && sr % 4 == 0 && K % 4 == 0) return 1;
  if (al && sr == 1 && sk % 4 == 0 && nrows % 4 == 0) return 2;
  return 0;
}

// NV float4 of an R x BK operand tile: rows [r0, r0 + R), k in [kk, kk + BK); rows >= nrows and
// k >= k1 read as zero (mode 1 / 2: a vector is inside or outside as a whole, k1 and nrows being
// multiples of 4 there)
template <int R, int BK, int NV>
__device__ __forceinline__ void m_opnd_load(const float* P, int64_t sr, int64_t sk, int nrows, int r0, int kk, int k1,
                                            int mode, float scale, f4 (&v)[NV]) {
  const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int i = 0; i < NV; i++) {
    const int e = threadIdx.x + 256 * i;
    if (mode == 2) {
      const int gr = r0 + (e % (R / 4)) * 4, gk = kk + e / (R / 4);
      v[i] = (gr < nrows && gk < k1) ? *reinterpret_cast<const f4*>(P + (int64_t)gk * sk + gr) : zero;
    } else {
      const int gr = r0 + e / (BK / 4), gk = kk + (e % (BK / 4)) * 4;
      if (mode == 1) {
        v[i] = (gr < nrows && gk < k1) ? *reinterpret_cast<const f4*>(P + (int64_t)gr * sr + gk) : zero;
      } else {
#pragma unroll
        for (int q = 0; q < 4; q++)
          v[i][q] = (gr < nrows && gk + q < k1) ? P[(int64_t)gr * sr + (int64_t)(gk + q) * sk] : 0.0f;
      }
    }
    if (scale != 1.0f)
#pragma unroll
      for (int q = 0; q < 4; q++) v[i][q] = v[i][q] * scale;
  }
}

// the same for a TQ8_0 operand: element (r, k) = Sc[e / 32] * Q[e], e = r * sr + k * sk (four
// consecutive codes of a vector share one 32-code scale block: e is a multiple of 4 there)
__device__ __forceinline__ int m_q8_mode(const int8_t* Q, int64_t sr, int64_t sk, int nrows, int K) {
  const bool al = (reinterpret_cast<uintptr_t>(Q) & 3u) == 0;
  if (al && sk == 1 && sr % 4 == 0 && K % 4 == 0) return 1;
  if (al && sr == 1 && sk % 4 == 0 && nrows % 4 == 0) return 2;
  return 0;
}
__device__ __forceinline__ f4 m_q8_vec(const int8_t* Q, const float* Sc, int64_t e) {
  const uint32_t u = *reinterpret_cast<const uint32_t*>(Q + e);
  const float d = Sc[e >> 5];
  return f4{d * (float)(int8_t)(u & 0xffu), d * (float)(int8_t)((u >> 8) & 0xffu), d * (float)(int8_t)((u >> 16) & 0xffu),
            d * (float)(int8_t)(u >> 24)};
}
template <int R, int BK, int NV>
__device__ __forceinline__ void m_opnd_load_q8(const int8_t* Q, const float* Sc, int64_t sr, int64_t sk, int nrows,
                                               int r0, int kk, int k1, int mode, f4 (&v)[NV]) {
  const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int i = 0; i < NV; i++) {
    const int e = threadIdx.x + 256 * i;
    if (mode == 2) {
      const int gr = r0 + (e % (R / 4)) * 4, gk = kk + e / (R / 4);
      v[i] = (gr < nrows && gk < k1) ? m_q8_vec(Q, Sc, (int64_t)gk * sk + gr) : zero;
    } else {
      const int gr = r0 + e / (BK / 4), gk = kk + (e % (BK / 4)) * 4;
      if (mode == 1) {
        v[i] = (gr < nrows && gk < k1) ? m_q8_vec(Q, Sc, (int64_t)gr * sr + gk) : zero;
      } else {
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int64_t ix = (int64_t)gr * sr + (int64_t)(gk + q) * sk;
          v[i][q] = (gr < nrows && gk + q < k1) ? Sc[ix >> 5] * (float)Q[ix] : 0.0f;
        }
      }
    }
  }
}

template <int R, int BK, int NV>
__device__ __forceinline__ void m_opnd_store(float* S, int mode, const f4 (&v)[NV]) {
#pragma unroll
  for (int i = 0; i < NV; i++) {
    const int e = threadIdx.x + 256 * i;
    if (mode == 2)
      *reinterpret_cast<f4*>(S + (e / (R / 4)) * (R + 4) + (e % (R / 4)) * 4) = v[i];
    else
      *reinterpret_cast<f4*>(S + (e / (BK / 4)) * (BK + 4) + (e % (BK / 4)) * 4) = v[i];
  }
}

// k = 16 kb + 4 g + q (q = 0..3) of LDS row r (mode 1 / 0 layout) or column r (mode 2)
template <int R, int BK>
__device__ __forceinline__ f4 m_opnd_frag(const float* S, int mode, int r, int kb, int g) {
  if (mode == 2) {
    const float* p = S + (16 * kb + 4 * g) * (R + 4) + r;
    return f4{p[0], p[R + 4], p[2 * (R + 4)], p[3 * (R + 4)]};
  }
  return *reinterpret_cast<const f4*>(S + r * (BK + 4) + 16 * kb + 4 * g);
}

template <int BM, bool BQ = false>
__device__ __forceinline__ void m_gemm(const MGemmArgs& a, int bx, int by, int bz) {
  using Cf = MGemmCfg<BM>;
  constexpr int BN = Cf::BN, BK = Cf::BK, TM = Cf::TM;
  __shared__ __attribute__((aligned(16))) float As[m_opnd_lds<BM, BK>()];
  __shared__ __attribute__((aligned(16))) float Bs[m_opnd_lds<BN, BK>()];
  const int b = bz, m0 = by * BM, n0 = bx * BN;
  if (a.causal == 1 && n0 > m0 + BM - 1) return;  // every element has n > m
  if (a.causal == 1 && a.live && !a.live[(m0 >> 6) * a.nlb + (n0 >> 6)]) return;  // no pair may attend
  const float* A = a.A + (int64_t)(b / a.divA) * a.sAb;
  const float* B = a.B + (int64_t)(b / a.divB) * a.sBb;
  int k0 = 0, k1 = a.K;
  if (a.causal == 2) k1 = min(a.K, m0 + BM);
  if (a.causal == 3) k0 = (m0 / BK) * BK;
  // packed layouts: k slabs (BK <= 64, inside one 64-block) of no live block are skipped
  const uint8_t* lrow = (a.live && a.causal >= 2) ? a.live + (a.causal == 2 ? (int64_t)(m0 >> 6) * a.nlb : (m0 >> 6))
                                                  : nullptr;
  const int lstep = a.causal == 2 ? 1 : a.nlb;
  auto next_live = [&](int kk) {
    if (lrow)
      while (kk < k1 && !lrow[(kk >> 6) * lstep]) kk += BK;
    return kk;
  };
  k0 = next_live(k0);
  const int amode = m_opnd_mode(A, a.sAm, a.sAk, a.sAb, a.M, a.K);
  const int8_t* Bq = reinterpret_cast<const int8_t*>(a.B);  // BQ: the codes (batch 1)
  const int bmode = BQ ? m_q8_mode(Bq, a.sBn, a.sBk, a.N, a.K) : m_opnd_mode(B, a.sBn, a.sBk, a.sBb, a.N, a.K);
  auto load_b = [&](int kk, f4 (&v)[Cf::NB]) {
    if constexpr (BQ)
      m_opnd_load_q8<BN, BK>(Bq, a.Bsc, a.sBn, a.sBk, a.N, n0, kk, k1, bmode, v);
    else
      m_opnd_load<BN, BK>(B, a.sBn, a.sBk, a.N, n0, kk, k1, bmode, 1.0f, v);
  };
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, li = lane & 15, g = lane >> 4;
  const int wm = (w >> 1) * (BM / 2), wn = (w & 1) * 32;
  f4 acc[TM][2];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) acc[i][j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  f4 ra[Cf::NA], rb[Cf::NB];
  if (k0 < k1) {
    m_opnd_load<BM, BK>(A, a.sAm, a.sAk, a.M, m0, k0, k1, amode, a.a_scale, ra);
    load_b(k0, rb);
  }
  for (int kk = k0; kk < k1;) {
    m_opnd_store<BM, BK>(As, amode, ra);
    m_opnd_store<BN, BK>(Bs, bmode, rb);
    __syncthreads();
    const int kn = next_live(kk + BK);
    if (kn < k1) {
      m_opnd_load<BM, BK>(A, a.sAm, a.sAk, a.M, m0, kn, k1, amode, a.a_scale, ra);
      load_b(kn, rb);
    }
#pragma unroll
    for (int kb = 0; kb < BK / 16; kb++) {
      f4 af[TM], bf[2];
#pragma unroll
      for (int i = 0; i < TM; i++) af[i] = m_opnd_frag<BM, BK>(As, amode, wm + 16 * i + li, kb, g);
#pragma unroll
      for (int j = 0; j < 2; j++) bf[j] = m_opnd_frag<BN, BK>(Bs, bmode, wn + 16 * j + li, kb, g);
#pragma unroll
      for (int q = 0; q < 4; q++)
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
          for (int j = 0; j < 2; j++) acc[i][j] = mfma_f32(af[i][q], bf[j][q], acc[i][j]);
    }
    __syncthreads();
    kk = kn;
  }
  float* C = a.C + (int64_t)b * a.sCb;
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int m = m0 + wm + 16 * i + 4 * g + e;
      if (m >= a.M) continue;
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const int n = n0 + wn + 16 * j + li;
        if (n >= a.N) continue;
        float* c = C + (int64_t)m * a.sCm + (int64_t)n * a.sCn;
        *c = a.accumulate ? *c + acc[i][j][e] : acc[i][j][e];
      }
    }
}

// Flat grids of 8 * ceil(n / 8) workgroups, XCD-aware: workgroup id goes to XCD id % 8, so the
// tile index l = (id % 8) * ceil(n / 8) + id / 8 gives each XCD a contiguous range of tiles (column
// tiles fastest, then row tiles, then batch): the tiles of one head share an XCD and its L2.  Row
// tiles run longest first (causal 2: the last rows reduce over the most k; causal 3: the first).
__device__ __forceinline__ int m_xcd_tile(int n) {
  const int per = (n + 7) / 8, id = blockIdx.x;
  const int l = (id & 7) * per + (id >> 3);
  return l < n ? l : -1;
}
template <int BM, bool BQ = false>
__device__ __forceinline__ void m_gemm_tile(const MGemmArgs& a, int l) {
  const int nx = (a.N + 63) / 64, ny = (a.M + BM - 1) / BM;
  const int bx = l % nx, yy = (l / nx) % ny, bz = l / (nx * ny);
  m_gemm<BM, BQ>(a, bx, a.causal == 2 ? ny - 1 - yy : yy, bz);
}
extern "C" __global__ __launch_bounds__(256) void rtq_m_gemm(MGemmArgs a) {
  const int l = m_xcd_tile((a.N + 63) / 64 * ((a.M + 63) / 64) * a.batch);
  if (l >= 0) m_gemm_tile<64>(a, l);
}
extern "C" __global__ __launch_bounds__(256) void rtq_m_gemm32(MGemmArgs a) {
  const int l = m_xcd_tile((a.N + 63) / 64 * ((a.M + 31) / 32) * a.batch);
  if (l >= 0) m_gemm_tile<32>(a, l);
}
// B a TQ8_0 weight (the trainer-native FrozenWeight::Q8_0 products of the runtime)
extern "C" __global__ __launch_bounds__(256) void rtq_m_gemm_q8(MGemmArgs a) {
  const int l = m_xcd_tile((a.N + 63) / 64 * ((a.M + 63) / 64) * a.batch);
  if (l >= 0) m_gemm_tile<64, true>(a, l);
}
extern "C" __global__ __launch_bounds__(256) void rtq_m_gemm32_q8(MGemmArgs a) {
  const int l = m_xcd_tile((a.N + 63) / 64 * ((a.M + 31) / 32) * a.batch);
  if (l >= 0) m_gemm_tile<32, true>(a, l);
}

// grouped products (MGemmGroupArgs) in one flat grid, so the products' workgroups share the CUs
__device__ __forceinline__ void m_gemm32_member(const MGemmArgs& a, int l) { m_gemm_tile<32>(a, l); }
extern "C" __global__ __launch_bounds__(256) void rtq_m_gemm32g(MGemmGroupArgs g) {
  const int id = m_xcd_tile(g.start[g.np]);
  if (id < 0) return;
  if (id < g.start[1])
    m_gemm32_member(g.p[0], id);
  else if (g.np > 1 && id < g.start[2])
    m_gemm32_member(g.p[1], id - g.start[1]);
  else if (g.np > 2 && id < g.start[3])
    m_gemm32_member(g.p[2], id - g.start[2]);
}

// ------------------------------------------------------------------ batched split-16-bit GEMM
// The attention products of m_gemm on 16-bit MFMA (16x16x32): each f32 operand element x is split
// as it is staged into a high and a low 16-bit part, and acc += Ah Bh + Al Bh + Ah Bl (f32
// accumulation).  HF (the forward's S = q k^T and o = p v): f16 parts rounded to nearest, hi =
// f16(x), lo = f16(x - hi), 22 significant bits, so the dropped Al Bl term leaves a relative error
// near 2^-22 per product (k and v, stored as f16 values, split exactly), close enough to f32 that
// the activations the next quantised linear sees keep their Q8 codes; the operands there are
// bounded (q scaled, probabilities, f16 k and v).  BF (the backward's products of score and output
// gradients, whose magnitudes can lie below f16's range): bf16 parts, each rounded to nearest, a
// relative error near 2^-16 per product.  Same tiles, grids, load modes, causal ranges and liveness skipping
// as m_gemm; LDS holds each operand as hi and lo planes [row][k] (k unit stride, rows padded to
// BK + 8 elements), so a lane's fragment (row li, k = 32 c + 8 g .. + 7) is one 16-byte read per
// plane (the padding puts the 16 rows of one lane group on distinct banks).  Mode-2 operands
// (unit stride along rows) are transposed as they are written (2-byte stores).
template <int R, int BK>
constexpr int m_bf_ld() { return BK + 8; }

// hi / lo bf16 halves of four floats, each rounded to nearest even (v_cvt_pk_bf16_f32; v - hi is
// exact in f32): hi + lo holds v within 2^-17 of |v|
__device__ __forceinline__ void m_split4(const f4 v, u2v& hi, u2v& lo) {
  uint32_t hb[4], lb[4];
#pragma unroll
  for (int c = 0; c < 4; c++) {
    const __bf16 h = (__bf16)v[c];
    hb[c] = __builtin_bit_cast(uint16_t, h);
    lb[c] = __builtin_bit_cast(uint16_t, (__bf16)(v[c] - (float)h));
  }
  hi.x = hb[0] | (hb[1] << 16);
  hi.y = hb[2] | (hb[3] << 16);
  lo.x = lb[0] | (lb[1] << 16);
  lo.y = lb[2] | (lb[3] << 16);
}

// the same split into f16 parts rounded to nearest
__device__ __forceinline__ void m_split4_f16(const f4 v, u2v& hi, u2v& lo) {
  uint32_t hb[4], lb[4];
#pragma unroll
  for (int c = 0; c < 4; c++) {
    const _Float16 h = (_Float16)v[c];
    hb[c] = __builtin_bit_cast(uint16_t, h);
    lb[c] = __builtin_bit_cast(uint16_t, (_Float16)(v[c] - (float)h));
  }
  hi.x = hb[0] | (hb[1] << 16);
  hi.y = hb[2] | (hb[3] << 16);
  lo.x = lb[0] | (lb[1] << 16);
  lo.y = lb[2] | (lb[3] << 16);
}

// NV float4 of an R x BK operand tile for m_gemm_bf: modes 0 / 1 as m_opnd_load; mode 2 (unit stride
// along rows) gives each thread one group of four rows at NV consecutive k (thread tid: rows
// 4 (tid % (R / 4)) .., k = NV (tid / (R / 4)) ..), so the store can write them transposed as
// runs along k
template <int R, int BK, int NV>
__device__ __forceinline__ void m_bf_load(const float* P, int64_t sr, int64_t sk, int nrows, int r0, int kk, int k1,
                                          int mode, float scale, f4 (&v)[NV]) {
  static_assert(NV * 1024 == R * BK, "every element of the tile once");
  if (mode != 2) {
    m_opnd_load<R, BK>(P, sr, sk, nrows, r0, kk, k1, mode, scale, v);
    return;
  }
  const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  const int gr = r0 + (threadIdx.x % (R / 4)) * 4, kb = kk + (threadIdx.x / (R / 4)) * NV;
#pragma unroll
  for (int i = 0; i < NV; i++) {
    const int gk = kb + i;
    v[i] = (gr < nrows && gk < k1) ? *reinterpret_cast<const f4*>(P + (int64_t)gk * sk + gr) : zero;
    if (scale != 1.0f)
#pragma unroll
      for (int q = 0; q < 4; q++) v[i][q] = v[i][q] * scale;
  }
}

template <int R, int BK, bool HF, int NV>
__device__ __forceinline__ void m_bf_store(uint16_t* Sh, uint16_t* Sl, int mode, const f4 (&v)[NV]) {
  constexpr int LD = m_bf_ld<R, BK>();
  u2v hi[NV], lo[NV];
#pragma unroll
  for (int i = 0; i < NV; i++) {
    if (HF)
      m_split4_f16(v[i], hi[i], lo[i]);
    else
      m_split4(v[i], hi[i], lo[i]);
  }
  if (mode == 2) {  // rows r .. r + 3 at k .. k + NV - 1: per row, NV consecutive elements
    static_assert(NV == 2 || NV == 4, "runs of 2 or 4 along k");
    const int r = (threadIdx.x % (R / 4)) * 4, k = (threadIdx.x / (R / 4)) * NV;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      // element q of each of the NV vectors: bf16 half (q & 1) of word q >> 1
      uint32_t eh[NV], el[NV];
#pragma unroll
      for (int i = 0; i < NV; i++) {
        const uint32_t wh = (q >> 1) ? hi[i].y : hi[i].x, wl = (q >> 1) ? lo[i].y : lo[i].x;
        eh[i] = (q & 1) ? (wh >> 16) : (wh & 0xffffu);
        el[i] = (q & 1) ? (wl >> 16) : (wl & 0xffffu);
      }
      if constexpr (NV == 4) {
        *reinterpret_cast<u2v*>(Sh + (r + q) * LD + k) = u2v{eh[0] | (eh[1] << 16), eh[2] | (eh[3] << 16)};
        *reinterpret_cast<u2v*>(Sl + (r + q) * LD + k) = u2v{el[0] | (el[1] << 16), el[2] | (el[3] << 16)};
      } else {
        *reinterpret_cast<uint32_t*>(Sh + (r + q) * LD + k) = eh[0] | (eh[1] << 16);
        *reinterpret_cast<uint32_t*>(Sl + (r + q) * LD + k) = el[0] | (el[1] << 16);
      }
    }
  } else {  // row r, columns k .. k + 3
#pragma unroll
    for (int i = 0; i < NV; i++) {
      const int e = threadIdx.x + 256 * i;
      const int r = e / (BK / 4), k = (e % (BK / 4)) * 4;
      *reinterpret_cast<u2v*>(Sh + r * LD + k) = hi[i];
      *reinterpret_cast<u2v*>(Sl + r * LD + k) = lo[i];
    }
  }
}

template <int BM, bool HF>
__device__ __forceinline__ void m_gemm_bf(const MGemmArgs& a, int bx, int by, int bz) {
  using Cf = MGemmCfg<BM>;
  constexpr int BN = Cf::BN, BK = Cf::BK, TM = Cf::TM;
  constexpr int LDA = m_bf_ld<BM, BK>(), LDB = m_bf_ld<BN, BK>();
  static_assert(BK % 32 == 0, "k slabs of whole 32-deep MFMA steps");
  __shared__ __attribute__((aligned(16))) uint16_t Ah[BM * LDA], Al[BM * LDA];
  __shared__ __attribute__((aligned(16))) uint16_t Bh[BN * LDB], Bl[BN * LDB];
  const int b = bz, m0 = by * BM, n0 = bx * BN;
  if (a.causal == 1 && n0 > m0 + BM - 1) return;  // every element has n > m
  if (a.causal == 1 && a.live && !a.live[(m0 >> 6) * a.nlb + (n0 >> 6)]) return;  // no pair may attend
  const float* A = a.A + (int64_t)(b / a.divA) * a.sAb;
  const float* B = a.B + (int64_t)(b / a.divB) * a.sBb;
  int k0 = 0, k1 = a.K;
  if (a.causal == 2) k1 = min(a.K, m0 + BM);
  if (a.causal == 3) k0 = (m0 / BK) * BK;
  const uint8_t* lrow = (a.live && a.causal >= 2) ? a.live + (a.causal == 2 ? (int64_t)(m0 >> 6) * a.nlb : (m0 >> 6))
                                                  : nullptr;
  const int lstep = a.causal == 2 ? 1 : a.nlb;
  auto next_live = [&](int kk) {
    if (lrow)
      while (kk < k1 && !lrow[(kk >> 6) * lstep]) kk += BK;
    return kk;
  };
  k0 = next_live(k0);
  const int amode = m_opnd_mode(A, a.sAm, a.sAk, a.sAb, a.M, a.K);
  const int bmode = m_opnd_mode(B, a.sBn, a.sBk, a.sBb, a.N, a.K);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, li = lane & 15, g = lane >> 4;
  const int wm = (w >> 1) * (BM / 2), wn = (w & 1) * 32;
  f4 acc[TM][2];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) acc[i][j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  f4 ra[Cf::NA], rb[Cf::NB];
  if (k0 < k1) {
    m_bf_load<BM, BK>(A, a.sAm, a.sAk, a.M, m0, k0, k1, amode, a.a_scale, ra);
    m_bf_load<BN, BK>(B, a.sBn, a.sBk, a.N, n0, k0, k1, bmode, 1.0f, rb);
  }
  for (int kk = k0; kk < k1;) {
    m_bf_store<BM, BK, HF>(Ah, Al, amode, ra);
    m_bf_store<BN, BK, HF>(Bh, Bl, bmode, rb);
    __syncthreads();
    const int kn = next_live(kk + BK);
    if (kn < k1) {
      m_bf_load<BM, BK>(A, a.sAm, a.sAk, a.M, m0, kn, k1, amode, a.a_scale, ra);
      m_bf_load<BN, BK>(B, a.sBn, a.sBk, a.N, n0, kn, k1, bmode, 1.0f, rb);
    }
#pragma unroll
    for (int kc = 0; kc < BK / 32; kc++) {
      bf8 ah[TM], al[TM], bh[2], bl[2];
#pragma unroll
      for (int i = 0; i < TM; i++) {
        const int o = (wm + 16 * i + li) * LDA + 32 * kc + 8 * g;
        ah[i] = *reinterpret_cast<const bf8*>(Ah + o);
        al[i] = *reinterpret_cast<const bf8*>(Al + o);
      }
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const int o = (wn + 16 * j + li) * LDB + 32 * kc + 8 * g;
        bh[j] = *reinterpret_cast<const bf8*>(Bh + o);
        bl[j] = *reinterpret_cast<const bf8*>(Bl + o);
      }
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
          if (HF) {
            acc[i][j] = mfma_f16(__builtin_bit_cast(half8, ah[i]), __builtin_bit_cast(half8, bh[j]), acc[i][j]);
            acc[i][j] = mfma_f16(__builtin_bit_cast(half8, al[i]), __builtin_bit_cast(half8, bh[j]), acc[i][j]);
            acc[i][j] = mfma_f16(__builtin_bit_cast(half8, ah[i]), __builtin_bit_cast(half8, bl[j]), acc[i][j]);
          } else {
            acc[i][j] = mfma_bf16(ah[i], bh[j], acc[i][j]);
            acc[i][j] = mfma_bf16(al[i], bh[j], acc[i][j]);
            acc[i][j] = mfma_bf16(ah[i], bl[j], acc[i][j]);
          }
        }
    }
    __syncthreads();
    kk = kn;
  }
  float* C = a.C + (int64_t)b * a.sCb;
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int m = m0 + wm + 16 * i + 4 * g + e;
      if (m >= a.M) continue;
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const int n = n0 + wn + 16 * j + li;
        if (n >= a.N) continue;
        float* c = C + (int64_t)m * a.sCm + (int64_t)n * a.sCn;
        *c = a.accumulate ? *c + acc[i][j][e] : acc[i][j][e];
      }
    }
}

template <int BM, bool HF>
__device__ __forceinline__ void m_gemm_bf_tile(const MGemmArgs& a, int l) {
  const int nx = (a.N + 63) / 64, ny = (a.M + BM - 1) / BM;
  const int bx = l % nx, yy = (l / nx) % ny, bz = l / (nx * ny);
  m_gemm_bf<BM, HF>(a, bx, a.causal == 2 ? ny - 1 - yy : yy, bz);
}
extern "C" __global__ __launch_bounds__(256) void rtq_m_gemm_bf(MGemmArgs a) {
  const int l = m_xcd_tile((a.N + 63) / 64 * ((a.M + 63) / 64) * a.batch);
  if (l >= 0) m_gemm_bf_tile<64, false>(a, l);
}
extern "C" __global__ __launch_bounds__(256) void rtq_m_gemm32_bf(MGemmArgs a) {
  const int l = m_xcd_tile((a.N + 63) / 64 * ((a.M + 31) / 32) * a.batch);
  if (l >= 0) m_gemm_bf_tile<32, false>(a, l);
}
extern "C" __global__ __launch_bounds__(256) void rtq_m_gemm_hf(MGemmArgs a) {
  const int l = m_xcd_tile((a.N + 63) / 64 * ((a.M + 63) / 64) * a.batch);
  if (l >= 0) m_gemm_bf_tile<64, true>(a, l);
}
extern "C" __global__ __launch_bounds__(256) void rtq_m_gemm32_hf(MGemmArgs a) {
  const int l = m_xcd_tile((a.N + 63) / 64 * ((a.M + 31) / 32) * a.batch);
  if (l >= 0) m_gemm_bf_tile<32, true>(a, l);
}
extern "C" __global__ __launch_bounds__(256) void rtq_m_gemm32g_bf(MGemmGroupArgs g) {
  const int id = m_xcd_tile(g.start[g.np]);
  if (id < 0) return;
  if (id < g.start[1])
    m_gemm_bf_tile<32, false>(g.p[0], id);
  else if (g.np > 1 && id < g.start[2])
    m_gemm_bf_tile<32, false>(g.p[1], id - g.start[1]);
  else if (g.np > 2 && id < g.start[3])
    m_gemm_bf_tile<32, false>(g.p[2], id - g.start[2]);
}

// ------------------------------------------------------------------ attention softmax
// grid (ceil(t / 4), nh), 256 threads: one wave per row i of head h (wave reductions, no barriers),
// over j <= i: p = exp(s - max) / sum (0 for j > i).  Packed layouts (a.live): only the row's live
// 64-blocks are visited, one element per lane, and only pairs that may attend enter the max and the
// sum (their p is 0).
__device__ __forceinline__ bool m_may_attend(const MSoftArgs& a, int si, int i, int j) {
  return j <= i && j < a.t && (a.seg[j] == 0 || a.seg[j] == si);
}

extern "C" __global__ __launch_bounds__(256) void rtq_m_softmax(MSoftArgs a) {
  const int i = blockIdx.x * 4 + (threadIdx.x >> 6), h = blockIdx.y, lane = threadIdx.x & 63;
  if (i >= a.t) return;  // whole wave
  float* row = a.s + ((int64_t)h * a.t + i) * a.t;
  float m = -__builtin_inff();
  if (a.live) {
    const uint8_t* lr = a.live + (int64_t)(i >> 6) * a.nlb;
    const int si = a.seg[i];
    for (int jb = 0; jb <= (i >> 6); jb++) {
      if (!lr[jb]) continue;
      const int j = jb * 64 + lane;
      if (m_may_attend(a, si, i, j)) m = fmaxf(m, row[j]);
    }
    m = wave_max(m);
    float s = 0.0f;
    for (int jb = 0; jb <= (i >> 6); jb++) {
      if (!lr[jb]) continue;
      const int j = jb * 64 + lane;
      if (m_may_attend(a, si, i, j)) s = s + expf(row[j] - m);
    }
    s = wave_sum(s);
    const float inv = __fdiv_rn(1.0f, s);
    for (int jb = 0; jb < a.nlb; jb++) {
      if (!lr[jb]) continue;
      const int j = jb * 64 + lane;
      if (j < a.t) row[j] = m_may_attend(a, si, i, j) ? expf(row[j] - m) * inv : 0.0f;
    }
    return;
  }
  for (int j = lane; j <= i; j += 64) m = fmaxf(m, row[j]);
  m = wave_max(m);
  float s = 0.0f;
  for (int j = lane; j <= i; j += 64) s = s + expf(row[j] - m);
  s = wave_sum(s);
  const float inv = __fdiv_rn(1.0f, s);
  for (int j = lane; j < a.t; j += 64) row[j] = j <= i ? expf(row[j] - m) * inv : 0.0f;
}

// grid (ceil(t / 4), nh), one wave per row: dS = (P (dP - sum_j P dP)) scale over j <= i, 0 beyond,
// written over dP (packed layouts: over the row's live blocks, 0 where a pair may not attend)
extern "C" __global__ __launch_bounds__(256) void rtq_m_softmax_bwd(MSoftArgs a) {
  const int i = blockIdx.x * 4 + (threadIdx.x >> 6), h = blockIdx.y, lane = threadIdx.x & 63;
  if (i >= a.t) return;
  const float* p = a.p + ((int64_t)h * a.t + i) * a.t;
  float* dp = a.dp + ((int64_t)h * a.t + i) * a.t;
  float s = 0.0f;
  if (a.live) {
    const uint8_t* lr = a.live + (int64_t)(i >> 6) * a.nlb;
    const int si = a.seg[i];
    for (int jb = 0; jb <= (i >> 6); jb++) {
      if (!lr[jb]) continue;
      const int j = jb * 64 + lane;
      if (m_may_attend(a, si, i, j)) s = s + p[j] * dp[j];
    }
    s = wave_sum(s);
    for (int jb = 0; jb < a.nlb; jb++) {
      if (!lr[jb]) continue;
      const int j = jb * 64 + lane;
      if (j < a.t) dp[j] = m_may_attend(a, si, i, j) ? (p[j] * (dp[j] - s)) * a.scale : 0.0f;
    }
    return;
  }
  for (int j = lane; j <= i; j += 64) s = s + p[j] * dp[j];
  s = wave_sum(s);
  for (int j = lane; j < a.t; j += 64) dp[j] = j <= i ? (p[j] * (dp[j] - s)) * a.scale : 0.0f;
}

// dk / dv [t x nkv x hd] = sum over the group's heads (head order) of dkh / dvh [nh x t x hd]
extern "C" __global__ __launch_bounds__(256) void rtq_m_group_sum(MGroupArgs a) {
  const int64_t n = (int64_t)a.t * a.nkv * a.hd;
  const int grp = a.nh / a.nkv;
  for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < n; idx += (int64_t)gridDim.x * 256) {
    const int e = (int)(idx % a.hd);
    const int64_t ig = idx / a.hd;
    const int g = (int)(ig % a.nkv);
    const int64_t i = ig / a.nkv;
    float sk = 0.0f, sv = 0.0f;
    for (int h = g * grp; h < (g + 1) * grp; h++) {
      const int64_t o = ((int64_t)h * a.t + i) * a.hd + e;
      sk = sk + a.dkh[o];
      sv = sv + a.dvh[o];
    }
    a.dk[idx] = sk;
    a.dv[i * a.ldv + (int64_t)g * a.hd + e] = sv;
  }
}

// ------------------------------------------------------------------ elementwise
#define M_ELT_LOOP                                                                                       \
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < a.n; i += (int64_t)gridDim.x * 256) { \
    const int64_t rr = i / a.cols, cc = i % a.cols, ia = rr * a.lda + cc, ic = rr * a.ldc + cc,          \
                  iy = rr * a.ldy + cc;
// SwiGLU forward: y = silu(a) * b
extern "C" __global__ __launch_bounds__(256) void rtq_m_swiglu(MEltArgs a) {
  M_ELT_LOOP
    (void)ic;
    a.y[iy] = m_silu(a.a[ia]) * a.b[ia];
  }
}

// SwiGLU backward: dg = (dh u) silu'(g) -> y, du = dh silu(g) -> z  (a = g, b = u, c = dh)
extern "C" __global__ __launch_bounds__(256) void rtq_m_swiglu_bwd(MEltArgs a) {
  M_ELT_LOOP
    const float g = a.a[ia], u = a.b[ia], dh = a.c[ic];
    a.y[iy] = (dh * u) * m_silu_grad(g);
    a.z[iy] = dh * m_silu(g);
  }
}

// y = a + b, or a + (b + c) when c is given
extern "C" __global__ __launch_bounds__(256) void rtq_m_add(MEltArgs a) {
  M_ELT_LOOP
    a.y[iy] = a.c ? a.a[ia] + (a.b[ia] + a.c[ic]) : a.a[ia] + a.b[ia];
  }
}
#undef M_ELT_LOOP

// off-block entries of a fused adapter's gb are cleared (they are gradients of B entries that are
// structurally zero)
extern "C" __global__ __launch_bounds__(256) void rtq_m_lora_mask(MMaskArgs a) {
  const int64_t n = a.rows * a.rank;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t row = i / a.rank, col = i % a.rank;
    bool keep = false;
    for (int m = 0; m < a.nm; m++)
      if (row >= a.row0[m] && row < a.row0[m] + a.nrow[m]) keep = col >= a.col0[m] && col < a.col0[m] + a.r[m];
    if (!keep) a.gb[i] = 0.0f;
  }
}

#include "rtq_attn.hip"
#include "rtq_fa.hip"
