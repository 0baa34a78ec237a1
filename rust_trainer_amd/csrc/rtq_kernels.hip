// rtq_kernels.hip — gfx950 kernels of the frozen quantised-matmul path.
//
// Compiled to a code object (hipcc --genco --offload-arch=gfx950) that the runtime loads with
// hipModuleLoadData.  Every kernel is extern "C" and takes one argument block from rtq_kargs.h.
//
// Arithmetic contract (reference: src/rie.rs:74-124, src/linear.rs:73-121):
//  * activations are quantised to Q8_0 exactly as ggml's reference quantiser does;
//  * each 32-element block dot is an exact integer sum.  The integer codes are fed to the
//    f16 MFMA as exact small integers (|q8| <= 127, |q4| <= 8), every product is exact in the
//    f32 accumulator and so is the 32-term sum (|isum| <= 32*127*127 < 2^24): the MFMA output
//    *is* the integer block sum, with no i32->f32 conversion to pay;
//  * block sums are scaled by d_w * d_x in f32 (the epilogue order is unpinned in the reference);
//  * dx = dy . W runs on f16 MFMA: W dequantised in registers to f16 (one rounding of the exact
//    product d*q) and dy scaled per token row by an exact power of two into f16 range.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include "rtq_kargs.h"

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

enum { FMT_Q4_0 = 2, FMT_Q8_0 = 8, FMT_Q4_K = 12, FMT_Q6_K = 14 };

__device__ __forceinline__ f4 mfma_f16(half8 a, half8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f4 mfma_f32(float a, float b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ half8 as_half8(uint4 v) { return __builtin_bit_cast(half8, v); }
__device__ __forceinline__ uint32_t comp(const uint4& v, int j) {
  return j == 0 ? v.x : (j == 1 ? v.y : (j == 2 ? v.z : v.w));
}
__device__ __forceinline__ uint16_t hcomp(const uint2& v, int j) {
  const uint32_t w = (j < 2) ? v.x : v.y;
  return (uint16_t)((j & 1) ? (w >> 16) : (w & 0xffffu));
}

// four bytes b0..b3 (each < 256) -> two half2 words holding 1024 + b (exact f16 integers)
__device__ __forceinline__ uint32_t bytes01_to_h2(uint32_t v) {
  return (v & 0xffu) | ((v & 0xff00u) << 8) | 0x64006400u;
}
__device__ __forceinline__ uint32_t bytes23_to_h2(uint32_t v) {
  return ((v >> 16) & 0xffu) | ((v >> 8) & 0xff0000u) | 0x64006400u;
}
__device__ __forceinline__ half2v sub_h2(uint32_t bits, _Float16 c) {
  half2v h = __builtin_bit_cast(half2v, bits);
  half2v cc = {c, c};
  return h - cc;  // exact: small integers
}

// Q4_0 fragment: bytes 4g..4g+3 of the block -> codes (nibble - 8) of elements
// {4g..4g+3} (low nibbles) then {16+4g..16+4g+3} (high nibbles), as exact f16.
__device__ __forceinline__ half8 q4_0_frag(uint32_t w) {
  const uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
  const _Float16 c = (_Float16)1032.0f;
  half2v a0 = sub_h2(bytes01_to_h2(lo), c), a1 = sub_h2(bytes23_to_h2(lo), c);
  half2v a2 = sub_h2(bytes01_to_h2(hi), c), a3 = sub_h2(bytes23_to_h2(hi), c);
  half8 r = {a0[0], a0[1], a1[0], a1[1], a2[0], a2[1], a3[0], a3[1]};
  return r;
}

// int8 codes (two words: elements {4g..4g+3}, {16+4g..16+4g+3}) -> exact f16
__device__ __forceinline__ half8 q8_frag(uint32_t lo, uint32_t hi) {
  lo ^= 0x80808080u;  // u = q + 128
  hi ^= 0x80808080u;
  const _Float16 c = (_Float16)1152.0f;
  half2v a0 = sub_h2(bytes01_to_h2(lo), c), a1 = sub_h2(bytes23_to_h2(lo), c);
  half2v a2 = sub_h2(bytes01_to_h2(hi), c), a3 = sub_h2(bytes23_to_h2(hi), c);
  half8 r = {a0[0], a0[1], a1[0], a1[1], a2[0], a2[1], a3[0], a3[1]};
  return r;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
  return v;
}

// ============================================================== utility
extern "C" __global__ __launch_bounds__(256) void rtq_fill_zero(FillArgs a) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < a.n; i += (int64_t)gridDim.x * 256) a.p[i] = 0.0f;
}

// ============================================================== activation quantisation (Q8_0)
// One thread per (token, 32-element block).  ggml reference semantics:
// d = amax/127, id = d ? 1/d : 0, q = roundf(x*id) (ties away from zero), stored scale fp16(d).
extern "C" __global__ __launch_bounds__(256) void rtq_quant_q8_0(QuantArgs a) {
  const int nb = a.Kp / 32;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)a.Tp * nb) return;
  const int t = (int)(idx / nb), b = (int)(idx % nb);
  const bool valid = t < a.T && b * 32 < a.K;
  float v[32];
  float amax = 0.0f;
  if (valid) {
    const float4* src = reinterpret_cast<const float4*>(a.x + (int64_t)t * a.K + b * 32);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float4 q = src[i];
      v[4 * i] = q.x;
      v[4 * i + 1] = q.y;
      v[4 * i + 2] = q.z;
      v[4 * i + 3] = q.w;
    }
#pragma unroll
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
  } else {
#pragma unroll
    for (int i = 0; i < 32; i++) v[i] = 0.0f;
  }
  const float d = __fdiv_rn(amax, 127.0f);
  const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
  const _Float16 dh = (_Float16)d;
  a.xd[(int64_t)b * a.Tp + t] = valid ? (float)dh : 0.0f;
  _Float16 q[32];
#pragma unroll
  for (int i = 0; i < 32; i++) q[i] = (_Float16)roundf(__fmul_rn(v[i], id));
  const int kc = b >> 2, j = b & 3, tg = t >> 4;
  uint4* xa = reinterpret_cast<uint4*>(a.xa) + ((int64_t)(tg * (a.Kp / 128) + kc) * 4 + j) * 64;
#pragma unroll
  for (int g = 0; g < 4; g++) {
    half8 f = {q[4 * g], q[4 * g + 1], q[4 * g + 2], q[4 * g + 3],
               q[16 + 4 * g], q[17 + 4 * g], q[18 + 4 * g], q[19 + 4 * g]};
    xa[(t & 15) + 16 * g] = __builtin_bit_cast(uint4, f);
  }
}

// ============================================================== LoRA down-projection
// h[t][j] = sum_k x[t][k] * A[j][k]  (src/linear.rs:85, matmul_nt).  One wave per token,
// lanes stride over k, 16 adapter rows per pass, wave reduction per row.
extern "C" __global__ __launch_bounds__(256) void rtq_lora_down(LoraDownArgs a) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= a.T) return;
  const float* x = a.x + (int64_t)t * a.K;
  for (int j0 = 0; j0 < a.r; j0 += 16) {
    float acc[16];
#pragma unroll
    for (int j = 0; j < 16; j++) acc[j] = 0.0f;
    for (int k = lane; k < a.K; k += 64) {
      const float xv = x[k];
#pragma unroll
      for (int j = 0; j < 16; j++)
        if (j0 + j < a.r) acc[j] = fmaf(xv, a.A[(int64_t)(j0 + j) * a.K + k], acc[j]);
    }
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const float s = wave_sum(acc[j]);
      if (lane == 0 && j0 + j < a.r) a.h[(int64_t)t * a.r + j0 + j] = s;
    }
  }
}

// ============================================================== forward (Q4_0 / Q8_0)
// Workgroup tile 64 tokens x 64 weight rows, 4 waves of 32 x 32 (2 x 2 MFMA tiles of 16x16).
// Per 32-element block: one 16x16x32 f16 MFMA per tile gives the exact integer block sums,
// then acc += isum * (d_w * d_x).  Weights and activations are read straight from their
// fragment layouts (one 16-byte load per lane per fragment, fully coalesced).
template <int FMT>
struct WChunk;

template <>
struct WChunk<FMT_Q4_0> {
  uint4 q;
  __device__ __forceinline__ void load(const FwdArgs& a, int rg, int kc, int Kc, int lane) {
    q = reinterpret_cast<const uint4*>(a.wq)[(int64_t)(rg * Kc + kc) * 64 + lane];
  }
  __device__ __forceinline__ half8 frag(int j) const { return q4_0_frag(comp(q, j)); }
};

template <>
struct WChunk<FMT_Q8_0> {
  uint4 q[2];
  __device__ __forceinline__ void load(const FwdArgs& a, int rg, int kc, int Kc, int lane) {
    const uint4* p = reinterpret_cast<const uint4*>(a.wq) + (int64_t)(rg * Kc + kc) * 128;
    q[0] = p[lane];
    q[1] = p[64 + lane];
  }
  __device__ __forceinline__ half8 frag(int j) const {
    const uint4& v = q[j >> 1];
    return (j & 1) ? q8_frag(v.z, v.w) : q8_frag(v.x, v.y);
  }
};

template <int FMT, bool DBG>
__device__ __forceinline__ void fwd_q32(const FwdArgs& a) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int li = lane & 15, g = lane >> 4;
  const int Kc = a.Kp / 128;
  const int rg0 = (blockIdx.x * 64 + (w & 1) * 32) >> 4;
  const int tg0 = (blockIdx.y * 64 + (w >> 1) * 32) >> 4;
  const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  f4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int jn = 0; jn < 2; jn++) acc[i][jn] = zero;

  const uint4* XA = reinterpret_cast<const uint4*>(a.xa);
  for (int kc = 0; kc < Kc; ++kc) {
    WChunk<FMT> wc[2];
    uint2 wd[2];
#pragma unroll
    for (int ns = 0; ns < 2; ns++) {
      wc[ns].load(a, rg0 + ns, kc, Kc, lane);
      wd[ns] = reinterpret_cast<const uint2*>(a.wd)[(int64_t)(rg0 + ns) * Kc * 16 + kc * 16 + li];
    }
    uint4 xa[2][4];
    f4 xd[2][4];
#pragma unroll
    for (int ts = 0; ts < 2; ts++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        xa[ts][j] = XA[((int64_t)((tg0 + ts) * Kc + kc) * 4 + j) * 64 + lane];
        xd[ts][j] = *reinterpret_cast<const f4*>(a.xd + (int64_t)(kc * 4 + j) * a.Tp + (tg0 + ts) * 16 + 4 * g);
      }
#pragma unroll
    for (int j = 0; j < 4; j++) {
#pragma unroll
      for (int ns = 0; ns < 2; ns++) {
        const half8 bf = wc[ns].frag(j);
        const float dw = h2f(hcomp(wd[ns], j));
#pragma unroll
        for (int ts = 0; ts < 2; ts++) {
          const f4 c = mfma_f16(as_half8(xa[ts][j]), bf, zero);
          if (DBG) {
            const int n = (rg0 + ns) * 16 + li, b = kc * 4 + j, nb = a.K / 32;
#pragma unroll
            for (int i = 0; i < 4; i++) {
              const int t = (tg0 + ts) * 16 + 4 * g + i;
              if (t < a.T && n < a.N && b < nb) a.isums[((int64_t)t * a.N + n) * nb + b] = (int32_t)c[i];
            }
          }
#pragma unroll
          for (int i = 0; i < 4; i++) acc[ts][ns][i] = fmaf(c[i], dw * xd[ts][j][i], acc[ts][ns][i]);
        }
      }
    }
  }

  // epilogue: y = acc (+ bias) (+ s * h.B^T), in the order of src/linear.rs:76-90
#pragma unroll
  for (int ts = 0; ts < 2; ts++)
#pragma unroll
    for (int ns = 0; ns < 2; ns++) {
      const int n = (rg0 + ns) * 16 + li;
      f4 lacc = zero;
      if (a.h) {
        const int trow = (tg0 + ts) * 16 + li;
        for (int j0 = 0; j0 < a.r; j0 += 4) {
          const int j = j0 + g;
          const float hv = (trow < a.T && j < a.r) ? a.h[(int64_t)trow * a.r + j] : 0.0f;
          const float bv = (n < a.N && j < a.r) ? a.lb[(int64_t)n * a.r + j] : 0.0f;
          lacc = mfma_f32(hv, bv, lacc);
        }
      }
      if (n < a.N) {
        const float bias = a.bias ? a.bias[n] : 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int t = (tg0 + ts) * 16 + 4 * g + i;
          if (t < a.T) {
            float v = acc[ts][ns][i];
            if (a.bias) v = v + bias;
            if (a.h) v = v + a.s * lacc[i];
            a.y[(int64_t)t * a.N + n] = v;
          }
        }
      }
    }
}

extern "C" __global__ __launch_bounds__(256) void rtq_fwd_q4_0(FwdArgs a) { fwd_q32<FMT_Q4_0, false>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_fwd_q8_0(FwdArgs a) { fwd_q32<FMT_Q8_0, false>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_fwd_q4_0_isums(FwdArgs a) { fwd_q32<FMT_Q4_0, true>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_fwd_q8_0_isums(FwdArgs a) { fwd_q32<FMT_Q8_0, true>(a); }

// ============================================================== backward: dy preparation
// One workgroup per (padded) token row: absmax -> exponent e with absmax*2^e in [2^14, 2^15),
// f16 fragments of dy*2^e (exact scaling, one RNE rounding), einv = 2^-e.
extern "C" __global__ __launch_bounds__(256) void rtq_dy_prep(DyPrepArgs a) {
  __shared__ float red[4];
  const int t = blockIdx.x, tid = threadIdx.x;
  const bool valid = t < a.T;
  if (valid && a.zero_dx)
    for (int k = tid; k < a.K; k += 256) a.zero_dx[(int64_t)t * a.K + k] = 0.0f;
  if (valid && a.zero_g)
    for (int j = tid; j < a.r; j += 256) a.zero_g[(int64_t)t * a.r + j] = 0.0f;
  const float* row = a.dy + (int64_t)t * a.N;
  float m = 0.0f;
  if (valid)
    for (int n = tid; n < a.N; n += 256) m = fmaxf(m, fabsf(row[n]));
  m = wave_max(m);
  if ((tid & 63) == 0) red[tid >> 6] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  int e = 0;
  if (m > 0.0f && m <= 3.4e38f) {
    int ex;
    frexpf(m, &ex);
    e = 15 - ex;
    e = e < -100 ? -100 : (e > 100 ? 100 : e);
  }
  const float sc = ldexpf(1.0f, e);
  if (tid == 0) a.einv[t] = ldexpf(1.0f, -e);
  const int ng = a.Np / 8;
  uint4* out = reinterpret_cast<uint4*>(a.dy16) + (int64_t)(t >> 4) * (a.Np / 32) * 64;
  for (int q = tid; q < ng; q += 256) {
    const int n8 = q * 8;
    _Float16 hv[8];
#pragma unroll
    for (int s = 0; s < 8; s++) {
      const int n = n8 + s;
      hv[s] = (_Float16)((valid && n < a.N) ? row[n] * sc : 0.0f);
    }
    half8 f = {hv[0], hv[1], hv[2], hv[3], hv[4], hv[5], hv[6], hv[7]};
    const int nc = n8 >> 5, gg = (n8 & 31) >> 3;
    out[nc * 64 + (t & 15) + 16 * gg] = __builtin_bit_cast(uint4, f);
  }
}

// ============================================================== LoRA g = s * dy . B
// One wave per (16 tokens, split of n, 16 adapter columns); f32 MFMA 16x16x4 over n; atomics.
extern "C" __global__ __launch_bounds__(64) void rtq_lora_g(LoraGArgs a) {
  const int lane = threadIdx.x, li = lane & 15, g = lane >> 4;
  const int t0 = blockIdx.x * 16, j0 = blockIdx.z * 16;
  const int n0 = blockIdx.y * a.n_per_split;
  const int n1 = min(n0 + a.n_per_split, a.N);
  const int trow = t0 + li, jcol = j0 + li;
  f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int n = n0; n < n1; n += 4) {
    const int nn = n + g;
    const float av = (trow < a.T && nn < n1) ? __fmul_rn(a.dy[(int64_t)trow * a.N + nn], a.s) : 0.0f;
    const float bv = (jcol < a.r && nn < n1) ? a.lb[(int64_t)nn * a.r + jcol] : 0.0f;
    acc = mfma_f32(av, bv, acc);
  }
  if (jcol < a.r)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int t = t0 + 4 * g + i;
      if (t < a.T) atomicAdd(&a.g[(int64_t)t * a.r + jcol], acc[i]);
    }
}

// ============================================================== dx = dy . W (+ g . A)
// Workgroup tile 64 tokens x 128 columns (one K chunk), rows of W split over blockIdx.z.
// Per 32-row step the 32 x 128 weight slab is dequantised to f16 (d*q, one rounding) and
// stored transposed in LDS ([k][n]) so each lane reads its B fragment (8 consecutive rows of
// one column) with one 16-byte LDS read; dy fragments come straight from global memory.
template <int FMT>
__device__ __forceinline__ void dx_dequant_store(const DxArgs& a, _Float16 (*wt)[40], int rg, int kc, int Kc,
                                                 int tid);

template <>
__device__ __forceinline__ void dx_dequant_store<FMT_Q4_0>(const DxArgs& a, _Float16 (*wt)[40], int rg0, int kc,
                                                           int Kc, int tid) {
  const int rgi = tid >> 7, ll = (tid & 127) >> 1, part = tid & 1;
  const int rg = rg0 + rgi;
  const uint2 q = reinterpret_cast<const uint2*>(a.wq)[((int64_t)(rg * Kc + kc) * 64 + ll) * 2 + part];
  const uint32_t d2 = reinterpret_cast<const uint32_t*>(a.wd)[((int64_t)(rg * Kc + kc) * 16 + (ll & 15)) * 2 + part];
  const int nl = rgi * 16 + (ll & 15), gg = ll >> 4;
#pragma unroll
  for (int jj = 0; jj < 2; jj++) {
    const int j = 2 * part + jj;
    const uint32_t w = jj ? q.y : q.x;
    const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t)(jj ? (d2 >> 16) : (d2 & 0xffffu)));
    const half8 c = q4_0_frag(w);
#pragma unroll
    for (int s = 0; s < 4; s++) {
      wt[32 * j + 4 * gg + s][nl] = c[s] * d;
      wt[32 * j + 16 + 4 * gg + s][nl] = c[4 + s] * d;
    }
  }
}

template <>
__device__ __forceinline__ void dx_dequant_store<FMT_Q8_0>(const DxArgs& a, _Float16 (*wt)[40], int rg0, int kc,
                                                           int Kc, int tid) {
  const int rgi = tid >> 7, ll = (tid & 127) >> 1, part = tid & 1;
  const int rg = rg0 + rgi;
  const uint4 q = reinterpret_cast<const uint4*>(a.wq)[(int64_t)(rg * Kc + kc) * 128 + part * 64 + ll];
  const uint32_t d2 = reinterpret_cast<const uint32_t*>(a.wd)[((int64_t)(rg * Kc + kc) * 16 + (ll & 15)) * 2 + part];
  const int nl = rgi * 16 + (ll & 15), gg = ll >> 4;
#pragma unroll
  for (int jj = 0; jj < 2; jj++) {
    const int j = 2 * part + jj;
    const half8 c = jj ? q8_frag(q.z, q.w) : q8_frag(q.x, q.y);
    const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t)(jj ? (d2 >> 16) : (d2 & 0xffffu)));
#pragma unroll
    for (int s = 0; s < 4; s++) {
      wt[32 * j + 4 * gg + s][nl] = c[s] * d;
      wt[32 * j + 16 + 4 * gg + s][nl] = c[4 + s] * d;
    }
  }
}

template <int FMT>
__device__ __forceinline__ void dx_q32(const DxArgs& a) {
  __shared__ __attribute__((aligned(16))) _Float16 wt[128][40];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, li = lane & 15, g = lane >> 4;
  const int kc = blockIdx.x, Kc = a.Kp / 128;
  const int tg0 = (blockIdx.y * 64 + (w >> 1) * 32) >> 4;
  const int kw = (w & 1) * 64;
  const int n0 = blockIdx.z * a.n_per_split;
  const int n1 = min(n0 + a.n_per_split, a.Np);
  const int Nc = a.Np / 32;
  const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  f4 acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = zero;
  const uint4* DY = reinterpret_cast<const uint4*>(a.dy16);
  for (int n = n0; n < n1; n += 32) {
    __syncthreads();
    dx_dequant_store<FMT>(a, wt, n >> 4, kc, Kc, tid);
    __syncthreads();
    uint4 af[2];
#pragma unroll
    for (int ts = 0; ts < 2; ts++) af[ts] = DY[((int64_t)(tg0 + ts) * Nc + (n >> 5)) * 64 + lane];
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
      const half8 bf = *reinterpret_cast<const half8*>(&wt[kw + ks * 16 + li][8 * g]);
#pragma unroll
      for (int ts = 0; ts < 2; ts++) acc[ts][ks] = mfma_f16(as_half8(af[ts]), bf, acc[ts][ks]);
    }
  }
  const bool lora = a.g != nullptr && blockIdx.z == 0;
#pragma unroll
  for (int ts = 0; ts < 2; ts++)
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
      const int k = kc * 128 + kw + ks * 16 + li;
      f4 lacc = zero;
      if (lora) {
        const int trow = (tg0 + ts) * 16 + li;
        for (int j0 = 0; j0 < a.r; j0 += 4) {
          const int j = j0 + g;
          const float gv = (trow < a.T && j < a.r) ? a.g[(int64_t)trow * a.r + j] : 0.0f;
          const float av = (k < a.K && j < a.r) ? a.la[(int64_t)j * a.K + k] : 0.0f;
          lacc = mfma_f32(gv, av, lacc);
        }
      }
      if (k < a.K)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int t = (tg0 + ts) * 16 + 4 * g + i;
          if (t < a.T) {
            float v = acc[ts][ks][i] * a.einv[t];
            if (lora) v += lacc[i];
            atomicAdd(&a.dx[(int64_t)t * a.K + k], v);
          }
        }
    }
}

extern "C" __global__ __launch_bounds__(256) void rtq_dx_q4_0(DxArgs a) { dx_q32<FMT_Q4_0>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_dx_q8_0(DxArgs a) { dx_q32<FMT_Q8_0>(a); }

// ============================================================== LoRA gradients
// gb[n][j] += sum_t (s*dy[t][n]) h[t][j]   (matmul_tn_acc, src/linear.rs:109)
// ga[j][k] += sum_t g[t][j] x[t][k]        (matmul_tn_acc, src/linear.rs:113)
// One wave per 16x16 output tile, f32 MFMA 16x16x4 over t; each tile has a single writer.
extern "C" __global__ __launch_bounds__(64) void rtq_lora_grads(LoraGradArgs a) {
  const int lane = threadIdx.x, li = lane & 15, g = lane >> 4;
  const int jt = (a.r + 15) / 16;
  f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  if ((int)blockIdx.x < a.n_tiles_gb) {
    const int nt = blockIdx.x / jt, jtile = blockIdx.x % jt;
    const int nrow = nt * 16 + li, jcol = jtile * 16 + li;
    for (int t0 = 0; t0 < a.T; t0 += 4) {
      const int t = t0 + g;
      const float av = (nrow < a.N && t < a.T) ? __fmul_rn(a.dy[(int64_t)t * a.N + nrow], a.s) : 0.0f;
      const float bv = (jcol < a.r && t < a.T) ? a.h[(int64_t)t * a.r + jcol] : 0.0f;
      acc = mfma_f32(av, bv, acc);
    }
    if (jcol < a.r)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int n = nt * 16 + 4 * g + i;
        if (n < a.N) a.gb[(int64_t)n * a.r + jcol] += acc[i];
      }
  } else {
    const int b = blockIdx.x - a.n_tiles_gb;
    const int jtile = b % jt, kt = b / jt;
    const int jrow = jtile * 16 + li, kcol = kt * 16 + li;
    for (int t0 = 0; t0 < a.T; t0 += 4) {
      const int t = t0 + g;
      const float av = (jrow < a.r && t < a.T) ? a.g[(int64_t)t * a.r + jrow] : 0.0f;
      const float bv = (kcol < a.K && t < a.T) ? a.x[(int64_t)t * a.K + kcol] : 0.0f;
      acc = mfma_f32(av, bv, acc);
    }
    if (kcol < a.K)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int j = jtile * 16 + 4 * g + i;
        if (j < a.r) a.ga[(int64_t)j * a.K + kcol] += acc[i];
      }
  }
}

// ============================================================== row dequant (FrozenMatmul::row)
// One thread per (row, 32-element block); bit-exact ggml dequant: (q - 8) * d, q * d.
extern "C" __global__ __launch_bounds__(256) void rtq_rows_q4_0(RowArgs a) {
  const int nb = a.K / 32, Kc = a.Kp / 128;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)a.count * nb) return;
  const int rl = (int)(idx / nb), b = (int)(idx % nb);
  const int n = a.r0 + rl, rg = n >> 4, li = n & 15, kc = b >> 2, j = b & 3;
  const uint4* q = reinterpret_cast<const uint4*>(a.wq) + (int64_t)(rg * Kc + kc) * 64;
  const float d = h2f(a.wd[((int64_t)(rg * Kc + kc) * 16 + li) * 4 + j]);
  float* out = a.out + (int64_t)rl * a.K + b * 32;
#pragma unroll
  for (int gg = 0; gg < 4; gg++) {
    const uint32_t w = comp(q[li + 16 * gg], j);
#pragma unroll
    for (int s = 0; s < 4; s++) {
      const int byte = (w >> (8 * s)) & 0xff;
      out[4 * gg + s] = (float)((byte & 0xf) - 8) * d;
      out[16 + 4 * gg + s] = (float)((byte >> 4) - 8) * d;
    }
  }
}

extern "C" __global__ __launch_bounds__(256) void rtq_rows_q8_0(RowArgs a) {
  const int nb = a.K / 32, Kc = a.Kp / 128;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)a.count * nb) return;
  const int rl = (int)(idx / nb), b = (int)(idx % nb);
  const int n = a.r0 + rl, rg = n >> 4, li = n & 15, kc = b >> 2, j = b & 3;
  const uint4* q = reinterpret_cast<const uint4*>(a.wq) + (int64_t)(rg * Kc + kc) * 128 + (j >> 1) * 64;
  const float d = h2f(a.wd[((int64_t)(rg * Kc + kc) * 16 + li) * 4 + j]);
  float* out = a.out + (int64_t)rl * a.K + b * 32;
#pragma unroll
  for (int gg = 0; gg < 4; gg++) {
    const uint4 v = q[li + 16 * gg];
    const uint32_t lo = (j & 1) ? v.z : v.x, hi = (j & 1) ? v.w : v.y;
#pragma unroll
    for (int s = 0; s < 4; s++) {
      out[4 * gg + s] = (float)(int8_t)((lo >> (8 * s)) & 0xff) * d;
      out[16 + 4 * gg + s] = (float)(int8_t)((hi >> (8 * s)) & 0xff) * d;
    }
  }
}
