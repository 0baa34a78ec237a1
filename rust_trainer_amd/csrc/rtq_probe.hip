// rtq_probe.hip — instruction-mix probes for the forward kernels' choice of MFMA (bench.py
// --mfma-mix; built into its own code object, not part of librtq.so).
//
// The forward's block dot (src/rie.rs:74-82, ggml's vec_dot_q4_0_q8_0 / q8_0_q8_0) needs, per
// output element and 32-column block, an exact integer block sum and one multiply-add by the
// product of the two block scales.  Each probe is a wave loop over NT independent output tiles,
// operands in registers (an empty asm keeps them opaque, so nothing is hoisted), doing one block
// per tile per iteration in one of three forms:
//   f16:   v_mfma_f32_16x16x32_f16 on the integer codes (exact sums in f32) + 4 FMAs per lane;
//   i8:    v_mfma_i32_32x32x32_i8 (K = 32: one block) + 16 conversions and 16 FMAs per lane;
//   i8x64: v_mfma_i32_16x16x64_i8 with one block in half of K (the other half zero) + 4
//          conversions and 4 FMAs per lane;
// the same three without the scale epilogue (the MFMA ceilings), and three with the scale products
// formed in the loop (below).  Outputs are summed into out[] so no work is dead.
#include <hip/hip_runtime.h>

typedef _Float16 p_half8 __attribute__((ext_vector_type(8)));
typedef float p_f4 __attribute__((ext_vector_type(4)));
typedef float p_f16 __attribute__((ext_vector_type(16)));
typedef int p_i4 __attribute__((ext_vector_type(4)));
typedef int p_i16 __attribute__((ext_vector_type(16)));

struct ProbeArgs {
  const int* in;  // 4096 ints of operand seeds
  float* out;     // one float per thread
  int iters;
};

template <int NT, bool EPI>
__device__ __forceinline__ void probe_f16(const ProbeArgs& a) {
  const int lane = threadIdx.x & 63;
  p_half8 A[NT], B;
  p_f4 s[NT], acc[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) {
#pragma unroll
    for (int e = 0; e < 8; e++) A[t][e] = (_Float16)(a.in[(lane * 8 + e + 64 * t) & 4095] % 127);
#pragma unroll
    for (int e = 0; e < 4; e++) {
      s[t][e] = 1e-6f * (float)a.in[(lane + e + t) & 4095];
      acc[t][e] = 0.0f;
    }
  }
#pragma unroll
  for (int e = 0; e < 8; e++) B[e] = (_Float16)(a.in[(lane * 3 + e) & 4095] % 127);
  const p_f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int it = 0; it < a.iters; it++) {
    asm volatile("" : "+v"(B));
#pragma unroll
    for (int t = 0; t < NT; t++) {
      const p_f4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[t], B, EPI ? zero : acc[t], 0, 0, 0);
      if (EPI) {
#pragma unroll
        for (int e = 0; e < 4; e++) acc[t][e] = fmaf(c[e], s[t][e], acc[t][e]);
      } else {
        acc[t] = c;
      }
    }
  }
  float r = 0.0f;
#pragma unroll
  for (int t = 0; t < NT; t++) r += (acc[t][0] + acc[t][1]) + (acc[t][2] + acc[t][3]);
  a.out[blockIdx.x * blockDim.x + threadIdx.x] = r;
}

template <int NT, bool EPI>
__device__ __forceinline__ void probe_i8(const ProbeArgs& a) {
  const int lane = threadIdx.x & 63;
  p_i4 A[NT], B;
  p_f16 s[NT], acc[NT];
  p_i16 ci[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) {
#pragma unroll
    for (int e = 0; e < 4; e++) A[t][e] = a.in[(lane * 4 + e + 64 * t) & 4095];
#pragma unroll
    for (int e = 0; e < 16; e++) {
      s[t][e] = 1e-6f * (float)a.in[(lane + e + t) & 4095];
      acc[t][e] = 0.0f;
      ci[t][e] = 0;
    }
  }
#pragma unroll
  for (int e = 0; e < 4; e++) B[e] = a.in[(lane * 5 + e) & 4095];
  const p_i16 zero = {};
  for (int it = 0; it < a.iters; it++) {
    asm volatile("" : "+v"(B));
#pragma unroll
    for (int t = 0; t < NT; t++) {
      const p_i16 c = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[t], B, EPI ? zero : ci[t], 0, 0, 0);
      if (EPI) {
#pragma unroll
        for (int e = 0; e < 16; e++) acc[t][e] = fmaf((float)c[e], s[t][e], acc[t][e]);
      } else {
        ci[t] = c;
      }
    }
  }
  float r = 0.0f;
#pragma unroll
  for (int t = 0; t < NT; t++)
#pragma unroll
    for (int e = 0; e < 16; e++) r += EPI ? acc[t][e] : (float)ci[t][e];
  a.out[blockIdx.x * blockDim.x + threadIdx.x] = r;
}

template <int NT, bool EPI>
__device__ __forceinline__ void probe_i8x64(const ProbeArgs& a) {
  const int lane = threadIdx.x & 63;
  p_i4 A[NT], B;
  p_f4 s[NT], acc[NT];
  p_i4 ci[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) {
#pragma unroll
    for (int e = 0; e < 4; e++) {
      // lanes 32..63 hold the k half that is zero (one 32-column block per MFMA)
      A[t][e] = lane < 32 ? a.in[(lane * 4 + e + 64 * t) & 4095] : 0;
      s[t][e] = 1e-6f * (float)a.in[(lane + e + t) & 4095];
      acc[t][e] = 0.0f;
      ci[t][e] = 0;
    }
  }
#pragma unroll
  for (int e = 0; e < 4; e++) B[e] = a.in[(lane * 5 + e) & 4095];
  const p_i4 zero = {0, 0, 0, 0};
  for (int it = 0; it < a.iters; it++) {
    asm volatile("" : "+v"(B));
#pragma unroll
    for (int t = 0; t < NT; t++) {
      const p_i4 c = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[t], B, EPI ? zero : ci[t], 0, 0, 0);
      if (EPI) {
#pragma unroll
        for (int e = 0; e < 4; e++) acc[t][e] = fmaf((float)c[e], s[t][e], acc[t][e]);
      } else {
        ci[t] = c;
      }
    }
  }
  float r = 0.0f;
#pragma unroll
  for (int t = 0; t < NT; t++)
#pragma unroll
    for (int e = 0; e < 4; e++) r += EPI ? acc[t][e] : (float)ci[t][e];
  a.out[blockIdx.x * blockDim.x + threadIdx.x] = r;
}

// The full per-block cost: the scale products d_w[row] * d_x[col] formed in the loop as well.
//   f16s: one 4-block f16 16x16x4 MFMA per token tile gives the products of 2 row groups x 2 blocks
//         (the forward kernels' arrangement), then per tile and block the f16 16x16x32 + 4 FMAs;
//   i8m:  per 32 x 32 tile and block an f16 32x32x8 MFMA (k slot 0 only) forms the 16 products of a
//         lane, then the i8 32x32x32 + 16 conversions + 16 FMAs;
//   i8v:  the 16 products by VALU (d_w of the lane's rows times d_x of its column), then as i8m.
typedef _Float16 p_half4 __attribute__((ext_vector_type(4)));
template <int NT>
__device__ __forceinline__ void probe_f16s(const ProbeArgs& a) {
  const int lane = threadIdx.x & 63;
  p_half8 A[NT], B;
  p_half4 SA, SB;
  p_f4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) {
#pragma unroll
    for (int e = 0; e < 8; e++) A[t][e] = (_Float16)(a.in[(lane * 8 + e + 64 * t) & 4095] % 127);
#pragma unroll
    for (int e = 0; e < 4; e++) acc[t][e] = 0.0f;
  }
#pragma unroll
  for (int e = 0; e < 8; e++) B[e] = (_Float16)(a.in[(lane * 3 + e) & 4095] % 127);
#pragma unroll
  for (int e = 0; e < 4; e++) {
    SA[e] = e == 0 ? (_Float16)(1e-3f * (float)(a.in[lane & 4095] % 100)) : (_Float16)0.0f;
    SB[e] = e == 0 ? (_Float16)(1e-3f * (float)(a.in[(lane + 7) & 4095] % 100)) : (_Float16)0.0f;
  }
  const p_f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  const p_f16 zero16 = {};
  for (int it = 0; it < a.iters; it++) {
    asm volatile("" : "+v"(B), "+v"(SB));
#pragma unroll
    for (int t0 = 0; t0 < NT; t0 += 4) {  // 4 tile-blocks (2 row groups x 2 blocks) per scale MFMA
      const p_f16 sc = __builtin_amdgcn_mfma_f32_16x16x4f16(SA, SB, zero16, 0, 0, 0);
#pragma unroll
      for (int t = t0; t < t0 + 4 && t < NT; t++) {
        const p_f4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[t], B, zero, 0, 0, 0);
#pragma unroll
        for (int e = 0; e < 4; e++) acc[t][e] = fmaf(c[e], sc[4 * (t - t0) + e], acc[t][e]);
      }
    }
  }
  float r = 0.0f;
#pragma unroll
  for (int t = 0; t < NT; t++) r += (acc[t][0] + acc[t][1]) + (acc[t][2] + acc[t][3]);
  a.out[blockIdx.x * blockDim.x + threadIdx.x] = r;
}

template <int NT, bool VALU_SCALES>
__device__ __forceinline__ void probe_i8s(const ProbeArgs& a) {
  const int lane = threadIdx.x & 63;
  p_i4 A[NT], B;
  p_half4 SA, SB;
  float dw[NT][16], dx;
  p_f16 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) {
#pragma unroll
    for (int e = 0; e < 4; e++) A[t][e] = a.in[(lane * 4 + e + 64 * t) & 4095];
#pragma unroll
    for (int e = 0; e < 16; e++) {
      acc[t][e] = 0.0f;
      dw[t][e] = 1e-3f * (float)(a.in[(lane + e + t) & 4095] % 100);
    }
  }
#pragma unroll
  for (int e = 0; e < 4; e++) {
    B[e] = a.in[(lane * 5 + e) & 4095];
    SA[e] = (e == 0 && lane < 32) ? (_Float16)(1e-3f * (float)(a.in[lane & 4095] % 100)) : (_Float16)0.0f;
    SB[e] = (e == 0 && lane < 32) ? (_Float16)(1e-3f * (float)(a.in[(lane + 7) & 4095] % 100)) : (_Float16)0.0f;
  }
  dx = 1e-3f * (float)(a.in[(lane + 11) & 4095] % 100);
  const p_i16 zero = {};
  const p_f16 zero16 = {};
  for (int it = 0; it < a.iters; it++) {
    asm volatile("" : "+v"(B), "+v"(SB), "+v"(dx));
#pragma unroll
    for (int t = 0; t < NT; t++) {
      p_f16 sc;
      if (VALU_SCALES) {
#pragma unroll
        for (int e = 0; e < 16; e++) sc[e] = dw[t][e] * dx;
      } else {
        sc = __builtin_amdgcn_mfma_f32_32x32x8f16(SA, SB, zero16, 0, 0, 0);
      }
      const p_i16 c = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[t], B, zero, 0, 0, 0);
#pragma unroll
      for (int e = 0; e < 16; e++) acc[t][e] = fmaf((float)c[e], sc[e], acc[t][e]);
    }
  }
  float r = 0.0f;
#pragma unroll
  for (int t = 0; t < NT; t++)
#pragma unroll
    for (int e = 0; e < 16; e++) r += acc[t][e];
  a.out[blockIdx.x * blockDim.x + threadIdx.x] = r;
}

// 8 independent 16 x 16 tiles (f16, i8x64) or 2 of 32 x 32 (i8): 2048 outputs per wave each
extern "C" __global__ __launch_bounds__(256) void rtq_probe_f16(ProbeArgs a) { probe_f16<8, true>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_probe_f16_mfma(ProbeArgs a) { probe_f16<8, false>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_probe_i8(ProbeArgs a) { probe_i8<2, true>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_probe_i8_mfma(ProbeArgs a) { probe_i8<2, false>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_probe_i8x64(ProbeArgs a) { probe_i8x64<8, true>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_probe_i8x64_mfma(ProbeArgs a) { probe_i8x64<8, false>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_probe_f16s(ProbeArgs a) { probe_f16s<8>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_probe_i8m(ProbeArgs a) { probe_i8s<2, false>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_probe_i8v(ProbeArgs a) { probe_i8s<2, true>(a); }
