// rtq_kargs.h — kernel argument blocks and device-layout constants shared by the host runtime
// (rtq_runtime.cpp) and the gfx950 kernels (rtq_kernels.hip).  Every kernel takes exactly one
// of these structs by value, so hipModuleLaunchKernel passes one parameter.
//
// Device weight layout ("row-group / K-chunk" layout, same byte count as GGUF):
//   rows are padded to Np = roundup(N, 64) and grouped by 16 (one MFMA tile edge); columns
//   are padded to Kp = roundup(K, 128) for Q4_0 / Q8_0 (a chunk = 4 blocks of 32) and to
//   roundup(K, 256) for Q4_K / Q6_K (a chunk = one 256-element super-block).  For every
//   (row group rg, chunk kc) the quant codes of the 16 rows are stored so that lane l of a
//   wave (row rg*16 + l%16, k-group g = l/16) reads its MFMA fragment with one coalesced
//   16-byte load: lane l holds, for every 32-element group j of the chunk, the codes of
//   elements {32j + 4g .. 32j + 4g + 3} and {32j + 16 + 4g .. 32j + 16 + 4g + 3}.  For Q4_0
//   that is exactly bytes 4g..4g+3 of the GGUF block (low nibbles: the first four, high
//   nibbles: the second four), so no nibble is moved across bytes.
#pragma once
#include <stdint.h>

#define RTQ_ROW_PAD 64     // Np multiple
#define RTQ_T_PAD 64       // Tp multiple (token tiles)
#define RTQ_CHUNK_Q 128    // K chunk of Q4_0 / Q8_0
#define RTQ_CHUNK_K 256    // K chunk of Q4_K / Q6_K

// ---------------------------------------------------------------- activation quantisation
// x [T x K] f32 -> MFMA A-operand fragments of the integer codes (as f16, exact) and scales.
//   xa: uint4 [Tp/16][Kp/32 blocks / 4 per chunk][4][64]  (one uint4 = 8 halves per lane)
//   xd: f32 [Kp/32][Tp]  (value of the fp16 scale; 0 for padding)
//   K-quant (Q8_K): xd is [Kp/256][Tp] (f32 d), xb: f16 bsums [Tp/16][Kp/256][64] (16 per
//   super-block, 16-element groups, as MFMA A fragments of a K=16 product)
struct QuantArgs {
  const float* x;
  int T, K, Tp, Kp;
  void* xa;
  float* xd;
  void* xb;  // Q8_K only
};

// h[t][j] = sum_k x[t][k] * A[j][k]   (LoRA down-projection, src/linear.rs:85)
struct LoraDownArgs {
  const float* x;
  const float* A;
  int T, K, r;
  float* h;  // [T x r]
};

// ---------------------------------------------------------------- forward GEMM
struct FwdArgs {
  const void* wq;       // quant codes, device layout
  const uint16_t* wd;   // fp16 scales, device layout (Q4_K: d,dmin pairs; Q6_K: d)
  const void* wx;       // extra per-format data (Q4_K 6-bit scales/mins, Q6_K int8 scales)
  int Np, Kp;
  const void* xa;       // activation fragments
  const float* xd;      // activation scales
  const void* xb;       // activation bsums (Q8_K)
  int Tp, T, N, K;
  float* y;             // [T x N]
  const float* bias;    // [N] or null
  const float* h;       // [T x r] or null (LoRA disabled)
  const float* lb;      // LoRA B [N x r]
  int r;
  float s;              // alpha / r
  int32_t* isums;       // debug: [T][N][isums_per_row] or null
};

// ---------------------------------------------------------------- backward
// dy [T x N] f32 -> f16 fragments scaled per token row by 2^e_t (exact power of two) for the
// dx product; einv[t] = 2^-e_t.  Optionally zero-fills dx (Linear::backward returns a fresh dx)
// and g (LoRA, accumulated with atomics afterwards).
struct DyPrepArgs {
  const float* dy;
  int T, N, Tp, Np;
  void* dy16;       // uint4 [Tp/16][Np/32][64]
  float* einv;      // [Tp]
  float* zero_dx;   // [T x K] or null
  int K;
  float* zero_g;    // [T x r] or null
  int r;
};

// g[t][j] += s * sum_n dy[t][n] * B[n][j]   (src/linear.rs:108-111), split over n
struct LoraGArgs {
  const float* dy;
  const float* lb;  // [N x r]
  int T, N, r;
  float s;
  int n_per_split;
  float* g;         // [T x r], pre-zeroed
};

struct DxArgs {
  const void* wq;
  const uint16_t* wd;
  const void* wx;
  int Np, Kp;
  const void* dy16;
  const float* einv;
  int Tp, T, K;
  int n_per_split;  // rows of W per split (multiple of 32)
  float* dx;        // [T x K], accumulated with atomics
  const float* g;   // LoRA g [T x r] or null
  const float* la;  // LoRA A [r x K]
  int r;
};

// gb[n][j] += sum_t (s*dy[t][n]) * h[t][j];  ga[j][k] += sum_t g[t][j] * x[t][k]
struct LoraGradArgs {
  const float* dy;
  const float* h;
  const float* g;
  const float* x;
  int T, N, K, r;
  float s;
  float* gb;  // [N x r]
  float* ga;  // [r x K]
  int n_tiles_gb;  // blocks [0, n_tiles_gb) do gb, the rest do ga
};

// rows [r0, r0+count) dequantised to f32 (bit-exact ggml dequant)
struct RowArgs {
  const void* wq;
  const uint16_t* wd;
  const void* wx;
  int Np, Kp, K;
  int r0, count;
  float* out;  // [count x K]
};

struct FillArgs {
  float* p;
  int64_t n;
};
