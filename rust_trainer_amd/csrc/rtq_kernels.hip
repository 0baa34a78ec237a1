// rtq_kernels.hip — gfx950 kernels of the frozen quantised-matmul path.
//
// Compiled to a code object (hipcc --genco --offload-arch=gfx950) that the runtime loads with
// hipModuleLoadData.  Every kernel is extern "C" and takes one argument block from rtq_kargs.h.
//
// Arithmetic contract (reference: src/rie.rs:74-124, src/linear.rs:73-121):
//  * activations are quantised to Q8_0 exactly as ggml's reference quantiser does;
//  * each 32-element block dot is an exact integer sum.  The integer codes are fed to the
//    f16 MFMA as exact small integers (|q8| <= 127, |q4| <= 8): every product is exact in the
//    f32 accumulator and so is the 32-term sum (|isum| <= 32*127*127 < 2^24), so the MFMA output
//    is the integer block sum itself, with no i32->f32 conversion to pay in the epilogue;
//    The int8 MFMA (rtq_mmi8_*) and v_dot4_i32_i8 (rtq_gemvq*, T <= 4) form the same integer sums;
//  * block sums are scaled by d_w * d_x in f32 (the epilogue order is unpinned in the reference);
//  * dx = dy . W at T = 1 (rtq_dxv1_*) multiplies in f32: the codes are exact f16 values, each
//    product fma(dy * scale, code, acc) by mixed-precision FMA;
//  * dx = dy . W (no dy quantisation, straight-through as in the reference) runs on f16 MFMA with
//    both operands split into hi + lo f16 parts: each dy row scaled by a power of two 2^e that
//    puts its largest |value| in [2^14, 2^15) (the whole row then lies in f16's range; the partial
//    is scaled back exactly), W's dequantised values split as hi = f16(d q), lo = the exact
//    residual (K-quants: of ggml's f32 value); dh.wh + dl.wh + dh.wl leaves a relative error near
//    2^-21 per product (the reference's f32 axpy, src/rie.rs:99-107: 2^-24);
//  * the LoRA products run on f32 MFMA (exact f32 products, f32 accumulation).
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include "rtq_kargs.h"

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
// native integer vectors (HIP's u4v/u2v are union-wrapped structs whose copies become memcpy
// and keep register arrays in scratch)
typedef uint32_t u4v __attribute__((ext_vector_type(4)));
typedef uint32_t u2v __attribute__((ext_vector_type(2)));

enum { FMT_Q4_0 = 2, FMT_Q8_0 = 8, FMT_Q4_K = 12, FMT_Q6_K = 14 };
__host__ __device__ constexpr bool is_kquant(int fmt) { return fmt == FMT_Q4_K || fmt == FMT_Q6_K; }
// formats whose device codes are bytes (Q8_0 layout); the others hold nibbles (Q4_0 layout)
__host__ __device__ constexpr bool byte_codes(int fmt) { return fmt == FMT_Q8_0 || fmt == FMT_Q6_K; }

__device__ __forceinline__ f4 mfma_f16(half8 a, half8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f4 mfma_bf16(bf8 a, bf8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f4 mfma_f32(float a, float b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
// v from the lane that DPP control CTRL names, within each row of 16 lanes (0xB1: lane ^ 1, 0x4E:
// lane ^ 2, 0x141: the mirror lane within each group of eight, 0x140: the mirror lane within the row)
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
// a raw buffer descriptor over [p, p + bytes): loads past the end return zero
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
// two floats -> f16 pair, rounded toward zero (v_cvt_pkrtz_f16_f32)
__device__ __forceinline__ half2v pk_rtz(float a, float b) {
  return __builtin_bit_cast(half2v, __builtin_amdgcn_cvt_pkrtz(a, b));
}
__device__ __forceinline__ uint32_t comp(const u4v& v, int j) {
  return j == 0 ? v.x : (j == 1 ? v.y : (j == 2 ? v.z : v.w));
}
__device__ __forceinline__ uint16_t hcomp(const u2v& v, int j) {
  const uint32_t w = (j < 2) ? v.x : v.y;
  return (uint16_t)((j & 1) ? (w >> 16) : (w & 0xffffu));
}

// Bytes b0..b3 of v -> two half2 words {1024 + b0, 1024 + b1}, {1024 + b2, 1024 + b3} (exact f16
// integers): v_perm_b32 interleaves the bytes with 0x64, the high byte of 1024.0 in f16.  The
// selector picks bytes 0-3 from the second operand and 4-7 from the first.
__device__ __forceinline__ uint32_t bytes01_to_h2(uint32_t v) { return __builtin_amdgcn_perm(0x64646464u, v, 0x04010400u); }
__device__ __forceinline__ uint32_t bytes23_to_h2(uint32_t v) { return __builtin_amdgcn_perm(0x64646464u, v, 0x04030402u); }
__device__ __forceinline__ half2v sub_h2(uint32_t bits, _Float16 c) {
  const half2v h = __builtin_bit_cast(half2v, bits);
  const half2v cc = {c, c};
  return h - cc;  // exact: small integers
}

// Q4_0 fragment: bytes 4g..4g+3 of the block -> codes (nibble - OFF) of elements
// {4g..4g+3} (low nibbles) then {16+4g..16+4g+3} (high nibbles), as exact f16.
template <int OFF = 8>
__device__ __forceinline__ half8 q4_0_frag(uint32_t w) {
  const uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
  const _Float16 c = (_Float16)(1024.0f + OFF);
  const half2v a0 = sub_h2(bytes01_to_h2(lo), c), a1 = sub_h2(bytes23_to_h2(lo), c);
  const half2v a2 = sub_h2(bytes01_to_h2(hi), c), a3 = sub_h2(bytes23_to_h2(hi), c);
  const half8 r = {a0[0], a0[1], a1[0], a1[1], a2[0], a2[1], a3[0], a3[1]};
  return r;
}

// int8 codes (two words: elements {4g..4g+3}, {16+4g..16+4g+3}) -> exact f16
__device__ __forceinline__ half8 q8_frag(uint32_t lo, uint32_t hi) {
  lo ^= 0x80808080u;  // u = q + 128
  hi ^= 0x80808080u;
  const _Float16 c = (_Float16)1152.0f;
  const half2v a0 = sub_h2(bytes01_to_h2(lo), c), a1 = sub_h2(bytes23_to_h2(lo), c);
  const half2v a2 = sub_h2(bytes01_to_h2(hi), c), a3 = sub_h2(bytes23_to_h2(hi), c);
  const half8 r = {a0[0], a0[1], a1[0], a1[1], a2[0], a2[1], a3[0], a3[1]};
  return r;
}


__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m));
  return v;
}

// ============================================================== utility
extern "C" __global__ __launch_bounds__(256) void rtq_fill_zero(FillArgs a) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < a.n; i += (int64_t)gridDim.x * 256) a.p[i] = 0.0f;
}

// grid-stride clear of rows [0, T) x [0, cols) by every thread of the grid
__device__ __forceinline__ void clear_rows(float* p, int64_t n) {
  const int64_t nthr = (int64_t)gridDim.x * gridDim.y * blockDim.x;
  const int64_t id = ((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * blockDim.x + threadIdx.x;
  for (int64_t i = id; i < n; i += nthr) p[i] = 0.0f;
}

// ============================================================== skinny f32 product
// out16x16 tile (rows r0.., cols c0..) of  P[row][col] = sum_k S[row][k] * M(col, k), reduced
// over k in [0, klen) by the NW waves of the workgroup (LDS reduction), f32 MFMA
// 16x16x4.  M(col, k) = Bm[col*ldb + k] when b_rows (row-major over k), else Bm[k*ldb + col]
// (column of a [klen x ncols] matrix).  Loads of four 16-k groups are issued before their
// MFMAs.  Leaves the reduced tile in red[NW*256 + row*16 + col] for the caller.
// Loads this lane's four consecutive k (kk .. kk+3) of S[row] and of M(col, .).  Indices are
// clamped into the matrices and out-of-range values replaced by 0, so every load is issued
// unconditionally (no divergent branches around memory instructions).
__device__ __forceinline__ void load_group(const float* S, int nrows, int lds, const float* Bm, int ncols, int ldb,
                                           bool b_rows, bool vec, int klen, int ke, int row, int col, int kk,
                                           float av[4], float bv[4]) {
  const uint32_t rowc = (uint32_t)min(row, nrows - 1), colc = (uint32_t)min(col, ncols - 1);
  const bool rin = row < nrows && kk < ke, cin = col < ncols && kk < ke;
  if (vec) {  // klen % 4 == 0, lds % 4 == 0, ldb % 4 == 0 (uniform)
    const uint32_t kc = (uint32_t)min(kk, klen - 4);
    const f4 q = *reinterpret_cast<const f4*>(S + (rowc * (uint32_t)lds + kc));
    av[0] = q.x; av[1] = q.y; av[2] = q.z; av[3] = q.w;
    if (b_rows) {
      const f4 r = *reinterpret_cast<const f4*>(Bm + (colc * (uint32_t)ldb + kc));
      bv[0] = r.x; bv[1] = r.y; bv[2] = r.z; bv[3] = r.w;
    } else {
#pragma unroll
      for (int c = 0; c < 4; c++) bv[c] = Bm[(kc + c) * (uint32_t)ldb + colc];
    }
#pragma unroll
    for (int c = 0; c < 4; c++) {
      av[c] = (rin && kk + c < klen) ? av[c] : 0.0f;
      bv[c] = (cin && kk + c < klen) ? bv[c] : 0.0f;
    }
  } else {
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const uint32_t k = (uint32_t)min(kk + c, klen - 1);
      const float x = S[rowc * (uint32_t)lds + k];
      const float y = b_rows ? Bm[colc * (uint32_t)ldb + k] : Bm[k * (uint32_t)ldb + colc];
      av[c] = (rin && kk + c < klen) ? x : 0.0f;
      bv[c] = (cin && kk + c < klen) ? y : 0.0f;
    }
  }
}

template <int NW>
__device__ __forceinline__ void skinny_tile(const float* S, int nrows, int lds, const float* Bm, int ncols, int ldb,
                                            bool b_rows, int klen, int r0, int c0, float sscale, float* red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, li = lane & 15, g = lane >> 4;
  const int per = ((klen + 15) / 16 + NW - 1) / NW * 16;  // k per wave, multiple of 16
  const int kb = w * per, ke = min(kb + per, klen);
  const int row = r0 + li, col = c0 + li;
  const bool vec = (klen & 3) == 0 && (lds & 3) == 0 && (ldb & 3) == 0 && klen >= 4;
  f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  // two batches of four 16-k groups in flight: the loads of batch U + 2 are issued right after
  // batch U's MFMAs (indices clamped, out-of-range values zeroed)
  float av[2][4][4], bv[2][4][4];
#define RTQ_SKINNY_LOAD(U, KB)                                                                           \
  _Pragma("unroll") for (int u = 0; u < 4; u++)                                                          \
      load_group(S, nrows, lds, Bm, ncols, ldb, b_rows, vec, klen, ke, row, col, (KB) + 16 * u + 4 * g,  \
                 av[U][u], bv[U][u]);
#define RTQ_SKINNY_MMA(U)                                                                                 \
  _Pragma("unroll") for (int u = 0; u < 4; u++) _Pragma("unroll") for (int c = 0; c < 4; c++) acc =     \
      mfma_f32(sscale == 1.0f ? av[U][u][c] : __fmul_rn(av[U][u][c], sscale), bv[U][u][c], acc);
  RTQ_SKINNY_LOAD(0, kb)
  RTQ_SKINNY_LOAD(1, kb + 64)
  for (int k = kb; k < ke; k += 128) {
    RTQ_SKINNY_MMA(0)
    RTQ_SKINNY_LOAD(0, k + 128)
    if (k + 64 < ke) {
      RTQ_SKINNY_MMA(1)
    }
    RTQ_SKINNY_LOAD(1, k + 192)
  }
#undef RTQ_SKINNY_MMA
#undef RTQ_SKINNY_LOAD
  // lane holds rows 4g+i, column li
#pragma unroll
  for (int i = 0; i < 4; i++) red[w * 256 + (4 * g + i) * 16 + li] = acc[i];
  __syncthreads();
  if (threadIdx.x < 256) {
    float s = 0.0f;
#pragma unroll
    for (int ww = 0; ww < NW; ww++) s += red[ww * 256 + threadIdx.x];
    red[threadIdx.x + NW * 256] = s;
  }
  __syncthreads();
}

// ============================================================== forward activation prep
// ggml Q8_0 reference semantics: d = amax/127, id = d ? 1/d : 0, q = roundf(x*id) (ties away
// from zero), stored scale fp16(d).
// ggml Q8_K reference semantics (K-quant weights, one 256-column super-block per token and
// workgroup): max = the signed element of largest |x| (the first one on ties), iscale = -127/max,
// q = min(127, nearest-even(iscale*x)), d = 1/iscale (f32); all zero: d = 0, q = 0.
// Grid (Tp/16, nq [+1]): workgroup (x, y < nq) quantises 16 tokens x RTQ_ACT_KQ columns, 256
// threads; thread (token tl = tid/16, segment sg = tid%16) owns 16 consecutive columns (half a
// block), so every load instruction of a wave covers four contiguous 1 KB row segments.
// With LoRA, workgroup (x, nq) computes h = x . A^T for its 16 tokens over all of K: per quarter
// the x and A tiles go through LDS to f32 MFMAs, the next quarter's tiles are loaded into registers
// while the current one is multiplied, and the four waves' column partials are summed in LDS.
__device__ __forceinline__ void load_seg(const float* p, bool ok, float v[16]) {
  if (ok) {
    const f4* src = reinterpret_cast<const f4*>(p);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const f4 q = src[i];
      v[4 * i] = q.x;
      v[4 * i + 1] = q.y;
      v[4 * i + 2] = q.z;
      v[4 * i + 3] = q.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; i++) v[i] = 0.0f;
  }
}

// (row n, rank j) lies in a member's block of a block-diagonal adapter (always, for a plain one)
// (member loops unrolled over the fixed capacity: constant indices keep the struct out of scratch)
__device__ __forceinline__ bool rb_keep(const RankBlocks& b, int n, int j) {
  if (b.nm == 0) return true;
  bool keep = false;
#pragma unroll
  for (int m = 0; m < 3; m++)
    if (m < b.nm && n >= b.row0[m] && n < b.row0[m] + b.nrow[m]) keep = j >= b.col0[m] && j < b.col0[m] + b.r[m];
  return keep;
}
// some (row, rank) pair of [n0, n1) x [j0, j1) lies in a member's block
__device__ __forceinline__ bool rb_any(const RankBlocks& b, int n0, int n1, int j0, int j1) {
  if (b.nm == 0) return true;
  bool any = false;
#pragma unroll
  for (int m = 0; m < 3; m++)
    any = any || (m < b.nm && max(n0, b.row0[m]) < min(n1, b.row0[m] + b.nrow[m]) &&
                  max(j0, b.col0[m]) < min(j1, b.col0[m] + b.r[m]));
  return any;
}

// ranks [lo, hi) that the LoRA up-projection of rows [n0, n1) reads: the span of their members'
// rank windows (every rank of a plain adapter; empty when no member row is adapted)
__device__ __forceinline__ void rb_span(const RankBlocks& b, int r, int n0, int n1, int& lo, int& hi) {
  if (b.nm == 0) {
    lo = 0;
    hi = r;
    return;
  }
  lo = r;
  hi = 0;
#pragma unroll
  for (int m = 0; m < 3; m++)
    if (m < b.nm && b.r[m] > 0 && max(n0, b.row0[m]) < min(n1, b.row0[m] + b.nrow[m])) {
      lo = min(lo, b.col0[m]);
      hi = max(hi, b.col0[m] + b.r[m]);
    }
  hi = max(hi, lo);
}

// LoRA-down partial product over a 256-column slice, by one 256-thread workgroup (f32 MFMA):
//   P[t][j] = sum over k in [k0, k0 + 256) of S[t][k] * M[j * ldm + k],  t in [t0, t0 + 16), j < r
// (h = x . A^T, src/linear.rs:85,106).  Written to out[(t * r + j) * pstride + pidx] (slice index
// fastest, so a consumer sums a token's partials in slice order with a few wide loads).  Columns
// beyond kend count as zero.  Thread (row tid / 16, segment tid % 16) holds 16 columns of one row
// of S and of one rank tile of M.

// thread (row tl, segment sg)'s 16 values of M's rank row j0 + tl, columns k0 + 16 sg .. (zero past
// r and kend)
__device__ __forceinline__ void lora_load_m(const float* M, int ldm, int r, int j0, int k0, int kend, float v[16]) {
  const int tid = threadIdx.x, jr = j0 + (tid >> 4), kk = k0 + (tid & 15) * 16;
  load_seg(M + (int64_t)jr * ldm + kk, jr < r && kk + 16 <= kend, v);
  if (jr < r && kk < kend && kk + 16 > kend) {
#pragma unroll
    for (int i = 0; i < 16; i++) v[i] = kk + i < kend ? M[(int64_t)jr * ldm + kk + i] : 0.0f;
  }
}

// The product for this thread's S values sv (its row's columns k0 + 16 sg .., zero past T and kend)
// and the first rank tile's M values mv (lora_load_m at j0 = 0, loaded by the caller so that they
// travel with its own loads); each next tile's loads are issued before the current one is contracted.
// NTOK = 8: sx already holds the 8 token rows (and zeros in rows 8 .. 15), sv is not read, and only
// tokens t0 .. t0 + 7 are written.
template <int NTOK = 16>
__device__ __forceinline__ void lora_partial_v(const float* sv, float mv[16], int T, const float* M, int ldm,
                                               int r, int k0, int kend, int t0, float* out, int pstride, int pidx,
                                               float* sx, float* sm, float* red) {
  constexpr int LDX = RTQ_ACT_KQ + 1;
  const int tid = threadIdx.x, tl = tid >> 4, sg = tid & 15;
  const int lane = tid & 63, w = tid >> 6, li = lane & 15, g = lane >> 4;
  if (NTOK == 16) {
#pragma unroll
    for (int i = 0; i < 16; i++) sx[tl * LDX + sg * 16 + i] = sv[i];
  }
  for (int j0 = 0; j0 < r; j0 += 16) {
#pragma unroll
    for (int i = 0; i < 16; i++) sm[tl * LDX + sg * 16 + i] = mv[i];
    if (j0 + 16 < r) lora_load_m(M, ldm, r, j0 + 16, k0, kend, mv);
    __syncthreads();
    f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < 16; u++) {
      const int kl = 64 * w + 4 * u + g;
      acc = mfma_f32(sx[li * LDX + kl], sm[li * LDX + kl], acc);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) red[w * 256 + (4 * g + i) * 16 + li] = acc[i];
    __syncthreads();
    {
      const int tt = tid >> 4, jj = tid & 15, ty = t0 + tt, jo = j0 + jj;
      const float ps = (red[tid] + red[256 + tid]) + (red[512 + tid] + red[768 + tid]);
      if (tt < NTOK && ty < T && jo < r) out[((int64_t)ty * r + jo) * pstride + pidx] = ps;
    }
    __syncthreads();
  }
}

__device__ __forceinline__ void lora_partial(const float* S, int T, int ks, const float* M, int ldm, int r, int k0,
                                             int kend, int t0, float* out, int pstride, int pidx, float* sx,
                                             float* sm, float* red) {
  const int tid = threadIdx.x, t = t0 + (tid >> 4), kk = k0 + (tid & 15) * 16;
  float v[16], mv[16];
  load_seg(S + (int64_t)t * ks + kk, t < T && kk + 16 <= kend, v);
  if (t < T && kk < kend && kk + 16 > kend) {  // ragged tail
#pragma unroll
    for (int i = 0; i < 16; i++) v[i] = kk + i < kend ? S[(int64_t)t * ks + kk + i] : 0.0f;
  }
  lora_load_m(M, ldm, r, 0, k0, kend, mv);
  lora_partial_v(v, mv, T, M, ldm, r, k0, kend, t0, out, pstride, pidx, sx, sm, red);
}

// LoRA-up input-gradient partial over one 256-row slice q of B (g = dy . B, src/linear.rs:111),
// for TW tokens t0 .. t0+TW-1, by one 256-thread workgroup (f32 MFMA):
//   gp[(q * T + t) * r + j] = sum over n in [256q, 256q + 256) of dy[t][n] * B[n][j]
// (slice-major, so each store instruction writes whole rank rows of consecutive tokens)
// B entries outside rb's blocks count as zero; rank tiles with none inside are written as zeros.
// B's slice (256 rows x 16 ranks) is staged in LDS once per rank tile and shared by the waves;
// LDS row n of the slice sits at 16n + 16 (n / 64), so the four lane groups of one MFMA step read
// four different 16-bank spans.  Each wave holds its dy rows in registers in MFMA operand order:
//   TW = 64: wave w owns tokens t0 + 16w .. +15 and all 256 rows; lane (token li, group g) loads
//            rows 64g .. 64g+63 of the slice (256 contiguous bytes), step u contracts row 64g + u;
//            no cross-wave reduction;
//   TW = 32: wave w = (wt, wh) = (w % 2, w / 2) owns tokens t0 + 16wt .. +15 and rows 128wh ..
//            128wh+127; lane (li, g) loads rows 128wh + 32g .. +31, step u contracts row
//            128wh + 32g + u; wave (wt, 0) adds wave (wt, 1)'s sums (through LDS) to its own;
//   TW = 16: wave w owns rows 64w .. 64w+63 of the 16 tokens; lane (li, g) loads rows
//            64w + 16g .. +15, step u contracts row 64w + 16g + u; the four waves' sums are added
//            in LDS in wave order (for grids too small to fill the chip with 64-token workgroups).
// thread tid's row k0 + tid of B, ranks j0 .. j0+15 (clamped addresses; masked when staged)
__device__ __forceinline__ void lora_load_b(const BwdPrepArgs& a, int k0, int j0, float bv[16]) {
  const float* brow = a.B + (int64_t)min(k0 + (int)threadIdx.x, a.N - 1) * a.r;
  if ((a.r & 3) == 0 && j0 + 16 <= a.r && (reinterpret_cast<uintptr_t>(a.B) & 15) == 0) {  // uniform
    const f4* b4 = reinterpret_cast<const f4*>(brow + j0);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const f4 e = b4[i];
      bv[4 * i] = e.x;
      bv[4 * i + 1] = e.y;
      bv[4 * i + 2] = e.z;
      bv[4 * i + 3] = e.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; i++) bv[i] = brow[min(j0 + i, a.r - 1)];
  }
}

template <int TW>
__device__ __forceinline__ void lora_up_partial(const BwdPrepArgs& a, int t0, int q, float* sb, float* red) {
  constexpr int KQ = RTQ_ACT_KQ, NU = TW;
  static_assert(KQ == 256, "one slice row per thread, four 64-row lane groups");
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, li = lane & 15, g = lane >> 4;
  const int wt = w & 1, wh = w >> 1;  // TW = 32
  const int k0 = q * KQ, tw = TW == 64 ? t0 + 16 * w : TW == 32 ? t0 + 16 * wt : t0, t = tw + li;
  // first slice row of this lane
  const int kl0 = TW == 64 ? 64 * g : TW == 32 ? 128 * wh + 32 * g : 64 * w + 16 * g, kb = k0 + kl0;
  float v[NU];
  {
    const float* row = a.dy + (int64_t)min(t, a.T - 1) * a.N;
    if (t < a.T && kb + NU <= a.N) {
      const f4* s4 = reinterpret_cast<const f4*>(row + kb);
#pragma unroll
      for (int i = 0; i < NU / 4; i++) {
        const f4 e = s4[i];
        v[4 * i] = e.x;
        v[4 * i + 1] = e.y;
        v[4 * i + 2] = e.z;
        v[4 * i + 3] = e.w;
      }
    } else {  // tokens past T, ragged N
#pragma unroll
      for (int u = 0; u < NU; u++) v[u] = (t < a.T && kb + u < a.N) ? row[min(kb + u, a.N - 1)] : 0.0f;
    }
  }
  const bool tok_ok = tw < a.T;  // wave-uniform
  // B's first rank tile travels with dy; each next one is loaded before the current one is contracted
  // (r = 0: the row maxima alone, B is null)
  float bv[16];
  bool any = a.r > 0 && rb_any(a.rb, k0, min(k0 + KQ, a.N), 0, min(16, a.r));  // uniform over the workgroup
  if (any) lora_load_b(a, k0, 0, bv);
  if (a.dymax) {  // max |dy| of each token over the slice: lane, then the four lane groups (then the waves)
    float mx = 0.0f;
#pragma unroll
    for (int u = 0; u < NU; u++) mx = fmaxf(mx, fabsf(v[u]));
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    if (TW == 64) {
      if (g == 0 && t < a.T) a.dymax[(int64_t)q * a.T + t] = mx;
    } else if (TW == 32) {
      if (g == 0) red[w * 16 + li] = mx;
      __syncthreads();
      if (tid < 32 && t0 + tid < a.T)  // token tid: waves (tid / 16, 0) and (tid / 16, 1)
        a.dymax[(int64_t)q * a.T + t0 + tid] = fmaxf(red[(tid >> 4) * 16 + (tid & 15)], red[((tid >> 4) + 2) * 16 + (tid & 15)]);
      // red is next written after the staging barrier below, which every reader has passed
    } else {
      if (g == 0) red[w * 16 + li] = mx;
      __syncthreads();
      if (tid < 16 && t0 + tid < a.T)
        a.dymax[(int64_t)q * a.T + t0 + tid] = fmaxf(fmaxf(red[tid], red[16 + tid]), fmaxf(red[32 + tid], red[48 + tid]));
      // red is next written after the staging barrier below, which every reader has passed
    }
  }
  for (int j0 = 0; j0 < a.r; j0 += 16) {
    f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    const bool cur = any;
    if (cur) {
      const int k = k0 + tid;
      float* dst = sb + 16 * tid + 16 * (tid >> 6);
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const int j = j0 + i;
        dst[i] = (k < a.N && j < a.r && rb_keep(a.rb, k, j)) ? bv[i] : 0.0f;
      }
    }
    if (j0 + 16 < a.r) {
      any = rb_any(a.rb, k0, min(k0 + KQ, a.N), j0 + 16, min(j0 + 32, a.r));
      if (any) lora_load_b(a, k0, j0 + 16, bv);
    }
    if (cur) {
      __syncthreads();
      if (tok_ok) {
        const float* sg = sb + 16 * kl0 + 16 * (kl0 >> 6) + li;
#pragma unroll
        for (int u = 0; u < NU; u++) acc = mfma_f32(v[u], sg[16 * u], acc);
      }
      if (TW == 16 || (TW == 32 && wh == 1)) {
#pragma unroll
        for (int i = 0; i < 4; i++) red[w * 256 + (4 * g + i) * 16 + li] = acc[i];
      }
      __syncthreads();  // red is complete; sb may be restaged (red is rewritten only after the next staging barrier)
      if (TW == 32 && wh == 0) {  // rows 0 .. 127, then rows 128 .. 255
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] = acc[i] + red[(w + 2) * 256 + (4 * g + i) * 16 + li];
      }
    }
    if (TW == 64 || (TW == 32 && wh == 0)) {  // lane (rank li, token group g) holds tokens tw + 4g + i
      const int j = j0 + li;
      if (j < a.r)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int tt = tw + 4 * g + i;
          if (tt < a.T) a.gp[((int64_t)q * a.T + tt) * a.r + j] = acc[i];
        }
    } else if (TW == 16) {  // thread (token tid / 16, rank tid % 16)
      const int tt = t0 + (tid >> 4), j = j0 + (tid & 15);
      const float ps = cur ? (red[tid] + red[256 + tid]) + (red[512 + tid] + red[768 + tid]) : 0.0f;
      if (tt < a.T && j < a.r) a.gp[((int64_t)q * a.T + tt) * a.r + j] = ps;
    }
  }
}

// sum of the np (multiple of 4) partials of element e, in slice order
__device__ __forceinline__ float sum_partials(const float* p, int64_t e, int np) {
  const f4* q = reinterpret_cast<const f4*>(p + e * np);
  float s = 0.0f;
  for (int i = 0; i < np / 4; i++) {
    const f4 v = q[i];
    s += ((v.x + v.y) + (v.z + v.w));
  }
  return s;
}

// the same sum over slice-major partials p[i * stride + e] (same association as sum_partials)
__device__ __forceinline__ float sum_slices(const float* p, int64_t e, int np, int64_t stride) {
  float s = 0.0f;
  for (int i = 0; i < np; i += 4) {
    const float* q = p + (int64_t)i * stride + e;
    s += ((q[0] + q[stride]) + (q[2 * stride] + q[3 * stride]));
  }
  return s;
}

// SiLU of the training step's MLP, x / (1 + e^-x) (src/tensor.rs:123-143; the decoder block's
// kernels use the same function)
__device__ __forceinline__ float rtq_silu(float x) { return __fdiv_rn(x, 1.0f + expf(-x)); }
__device__ __forceinline__ float rtq_sigmoid(float x) {
  if (x >= 0.0f) return __fdiv_rn(1.0f, 1.0f + expf(-x));
  const float e = expf(x);
  return __fdiv_rn(e, 1.0f + e);
}
__device__ __forceinline__ float rtq_silu_grad(float x) {
  const float s = rtq_sigmoid(x);
  return s * (1.0f + x * (1.0f - s));
}

template <bool QK>
__device__ __forceinline__ void act_prep(const ActArgs& a) {
  constexpr int KQ = RTQ_ACT_KQ, LDX = KQ + 1;
  __shared__ float sx[16 * LDX];
  __shared__ float sa[16 * LDX];
  __shared__ float red[4 * 256];
  const int tid = threadIdx.x, tl = tid >> 4, sg = tid & 15;
  const int t0 = blockIdx.x * 16, t = t0 + tl;
  const int Kc = a.Kp / 128;
  const int k0 = blockIdx.y * KQ;
  {
    const int kk = k0 + sg * 16;  // first column of this thread's segment
    float v[16], mv[16];
    if (a.A) lora_load_m(a.A, a.K, a.r, 0, k0, a.K, mv);  // uniform; in flight during the activation work
    if (a.na) {  // uniform: v = RMSNorm rows, in the order of rtq_m_rmsnorm's one-wave rows
      // wave w normalises rows t0 + 4w .. t0 + 4w + 3 whole (lane l: float4 columns 4l + 256i, i <
      // K / 256), then writes quarter blockIdx.y of each (x, nh) and passes it through LDS (sx) to
      // the thread layout below; quarters beyond K give zeros.  The 1 / rms is written once.
      // every load issued before any is used: addresses clamped into the rows (no branches between
      // the loads), out-of-range values replaced by zeros afterwards
      const int lane = tid & 63, w = tid >> 6, nv = a.K / 256, qy = blockIdx.y;
      const f4 z4 = {0.0f, 0.0f, 0.0f, 0.0f};
      const bool has_b = a.nb != nullptr;
      const float* pb = has_b ? a.nb : a.na;
      f4 wv[4], xv[4][4], bv[4][4];
#pragma unroll
      for (int i = 0; i < 4; i++) wv[i] = *reinterpret_cast<const f4*>(a.nw + 4 * lane + 256 * min(i, nv - 1));
#pragma unroll
      for (int rr = 0; rr < 4; rr++) {
        const int64_t ro = (int64_t)min(t0 + 4 * w + rr, a.T - 1) * a.K + 4 * lane;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          xv[rr][i] = *reinterpret_cast<const f4*>(a.na + ro + 256 * min(i, nv - 1));
          bv[rr][i] = *reinterpret_cast<const f4*>(pb + ro + 256 * min(i, nv - 1));
        }
      }
#pragma unroll
      for (int rr = 0; rr < 4; rr++) {
        const bool rin = t0 + 4 * w + rr < a.T;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const float xs = has_b ? xv[rr][i][e] + bv[rr][i][e] : xv[rr][i][e];
            xv[rr][i][e] = (rin && i < nv) ? xs : 0.0f;
          }
      }
#pragma unroll
      for (int rr = 0; rr < 4; rr++) {
        const int row = t0 + 4 * w + rr;
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++)
          if (i < nv)
#pragma unroll
            for (int e = 0; e < 4; e++) s = s + xv[rr][i][e] * xv[rr][i][e];
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, m);
        const float ir = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(s, (float)a.K) + a.neps));
        f4 y = z4;
#pragma unroll
        for (int i = 0; i < 4; i++)
          if (i < nv && i == qy) {
#pragma unroll
            for (int e = 0; e < 4; e++) y[e] = (xv[rr][i][e] * ir) * (wv[i][e] + a.noff);
            if (row < a.T) {
              const int64_t o = (int64_t)row * a.K + 256 * i + 4 * lane;
              if (a.nb) *reinterpret_cast<f4*>(a.nh + o) = xv[rr][i];
              *reinterpret_cast<f4*>(const_cast<float*>(a.x) + o) = y;
            }
          }
        if (qy == 0 && lane == 0 && row < a.T) a.ninv[row] = ir;
#pragma unroll
        for (int e = 0; e < 4; e++) sx[(4 * w + rr) * LDX + 4 * lane + e] = y[e];
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < 16; i++) v[i] = sx[tl * LDX + sg * 16 + i];
    } else if (a.sg) {  // uniform: v = silu(g) * u, written to x for the backward
      float gv[16], uv[16];
      load_seg(a.sg + (int64_t)t * a.ldsg + kk, t < a.T && kk < a.K, gv);
      load_seg(a.su + (int64_t)t * a.ldsg + kk, t < a.T && kk < a.K, uv);
#pragma unroll
      for (int i = 0; i < 16; i++) v[i] = rtq_silu(gv[i]) * uv[i];
      if (t < a.T && kk < a.K) {
        f4* xo = reinterpret_cast<f4*>(const_cast<float*>(a.x) + (int64_t)t * a.K + kk);
#pragma unroll
        for (int i = 0; i < 4; i++) xo[i] = f4{v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]};
      }
    } else {
      load_seg(a.x + (int64_t)t * a.K + kk, t < a.T && kk < a.K, v);  // K % 32 == 0: all in or all out
    }
    _Float16 q[16];  // codes: exact small integers
    float dstore;    // the block scale as the dot products use it
    if (!QK) {
      float amax = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; i++) amax = fmaxf(amax, fabsf(v[i]));
      amax = fmaxf(amax, __shfl_xor(amax, 1));  // the two halves of a block are adjacent lanes
      const float d = __fdiv_rn(amax, 127.0f);
      const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
#pragma unroll
      for (int i = 0; i < 16; i++) q[i] = (_Float16)roundf(__fmul_rn(v[i], id));
      dstore = (float)(_Float16)d;
    } else {
      // first element of largest |x| in this segment, then over the token's 16 adjacent lanes
      // (larger |x| wins, equal |x|: the lower column)
      float best = 0.0f, bmax = 0.0f;
      int bi = 0;
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const float ax = fabsf(v[i]);
        if (ax > best) {
          best = ax;
          bmax = v[i];
          bi = i;
        }
      }
      bi += sg * 16;
#pragma unroll
      for (int m = 1; m < 16; m <<= 1) {
        const float ob = __shfl_xor(best, m), om = __shfl_xor(bmax, m);
        const int oi = __shfl_xor(bi, m);
        if (ob > best || (ob == best && oi < bi)) {
          best = ob;
          bmax = om;
          bi = oi;
        }
      }
      const float iscale = best != 0.0f ? __fdiv_rn(-127.0f, bmax) : 0.0f;
#pragma unroll
      for (int i = 0; i < 16; i++) q[i] = (_Float16)fminf(127.0f, rintf(__fmul_rn(iscale, v[i])));
      dstore = best != 0.0f ? __fdiv_rn(1.0f, iscale) : 0.0f;
    }
    float csum = 0.0f;  // sum of the block's codes (exact integer), for the GEMV's seed
    if (a.xg) {         // uniform
#pragma unroll
      for (int i = 0; i < 16; i++) csum += (float)q[i];
      csum += __shfl_xor(csum, 1);
    }
    if (kk < a.Kp) {
      const int b = kk >> 5, hf = sg & 1, kc = b >> 2, j = b & 3;
      if (a.xq_i8) {  // uniform: int8 fragments of rtq_mmi8_*, k-group g at byte 8 (g % 2) + 4 hf of lane (t % 32) + 32 (g / 2)
        uint32_t* xq = reinterpret_cast<uint32_t*>(a.xq) + ((((int64_t)(t >> 5) * Kc + kc) * 4 + j) * 64 + (t & 31)) * 4 + hf;
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const uint32_t w = ((uint32_t)(int)q[4 * g] & 0xffu) | (((uint32_t)(int)q[4 * g + 1] & 0xffu) << 8) |
                             (((uint32_t)(int)q[4 * g + 2] & 0xffu) << 16) | ((uint32_t)(int)q[4 * g + 3] << 24);
          xq[(g >> 1) * 32 * 4 + (g & 1) * 2] = w;
        }
      } else {
      // this half block gives, for each k-group g, the four codes of one 8-element fragment half
      u2v* xq = reinterpret_cast<u2v*>(a.xq) + ((((int64_t)(t >> 4) * Kc + kc) * 4 + j) * 64 + (t & 15)) * 2 + hf;
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const half2v lo = {q[4 * g], q[4 * g + 1]}, hi = {q[4 * g + 2], q[4 * g + 3]};
        u2v w;
        w.x = __builtin_bit_cast(uint32_t, lo);
        w.y = __builtin_bit_cast(uint32_t, hi);
        xq[g * 16 * 2] = w;
      }
      }
      const bool real = t < a.T && kk < a.K;
      if (hf == 0) a.xd[((int64_t)kc * a.Tp + t) * 4 + j] = real ? dstore : 0.0f;
      if (a.xdh && hf == 0)  // Q8_0: dstore is an fp16 value
        a.xdh[((int64_t)kc * a.Tp + t) * 4 + j] = real ? __builtin_bit_cast(uint16_t, (_Float16)dstore) : (uint16_t)0;
      if (a.xg && hf == 0) {  // Tp == 16: t is the token within the tile
        a.xg[(int64_t)(b * 2) * 16 + t] = real ? dstore : 0.0f;
        a.xg[(int64_t)(b * 2 + 1) * 16 + t] = real ? -a.gbias * csum : 0.0f;
      }
    }
    // LoRA-down partial of these columns from the values in registers (zero past T and K, like the
    // codes; quarters beyond K write zero partials)
    if (a.A)  // uniform
      lora_partial_v(v, mv, a.T, a.A, a.K, a.r, k0, a.K, t0, a.hp, gridDim.y, blockIdx.y, sx, sa, red);
  }
  if (a.zero_y && blockIdx.y == 0) {
    for (int tt = 0; tt < 16; tt++) {
      const int ty = t0 + tt;
      if (ty < a.T)
        for (int n = tid; n < a.N; n += 256) a.zero_y[(int64_t)ty * a.N + n] = 0.0f;
    }
  }
}

extern "C" __global__ __launch_bounds__(256) void rtq_act_prep_q8_0(ActArgs a) { act_prep<false>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_act_prep_q8_k(ActArgs a) { act_prep<true>(a); }

// The block-norm activation kernel on NT-token tiles (NT = 8 or 4): 16 / NT times act_prep's
// workgroups for a given T, each reading NT rows whole for the sums of squares instead of 16.
// RMSNorm rows (NT / 4 per wave), Q8_0 codes as f16 fragments and the LoRA-down partials, each with
// act_prep's arithmetic in the same order, so the outputs carry the same bits.  Thread (token
// tl = tid / (256 / NT), segment sg) holds NT columns k0 + NT sg ..; the 32 / NT threads of a
// 32-column block are adjacent lanes.  Only for the norm input without the GEMV seed (xg), int8
// fragments, SwiGLU input or a y to zero.
template <int NT>
__device__ __forceinline__ void act_prep_norm(const ActArgs& a) {
  static_assert(NT == 8 || NT == 4, "8- or 4-token tiles");
  constexpr int TPT = 256 / NT, RPW = NT / 4, BL = 32 / NT;  // threads per token, rows per wave, lanes per block
  constexpr int KQ = RTQ_ACT_KQ, LDX = KQ + 1;
  __shared__ float sx[16 * LDX];
  __shared__ float sa[16 * LDX];
  __shared__ float red[4 * 256];
  const int tid = threadIdx.x, tl = tid / TPT, sg = tid % TPT;
  const int t0 = blockIdx.x * NT, t = t0 + tl;
  const int Kc = a.Kp / 128;
  const int k0 = blockIdx.y * KQ, kk = k0 + sg * NT;
  float mv[16];
  if (a.A) lora_load_m(a.A, a.K, a.r, 0, k0, a.K, mv);  // uniform; in flight during the norm
  {
    // wave w normalises rows t0 + RPW w .. t0 + RPW w + RPW - 1 whole (as act_prep, every load issued first)
    const int lane = tid & 63, w = tid >> 6, nv = a.K / 256, qy = blockIdx.y;
    const bool has_b = a.nb != nullptr;
    const float* pb = has_b ? a.nb : a.na;
    f4 wv[4], xv[RPW][4], bv[RPW][4];
#pragma unroll
    for (int i = 0; i < 4; i++) wv[i] = *reinterpret_cast<const f4*>(a.nw + 4 * lane + 256 * min(i, nv - 1));
#pragma unroll
    for (int rr = 0; rr < RPW; rr++) {
      const int64_t ro = (int64_t)min(t0 + RPW * w + rr, a.T - 1) * a.K + 4 * lane;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        xv[rr][i] = *reinterpret_cast<const f4*>(a.na + ro + 256 * min(i, nv - 1));
        bv[rr][i] = *reinterpret_cast<const f4*>(pb + ro + 256 * min(i, nv - 1));
      }
    }
#pragma unroll
    for (int rr = 0; rr < RPW; rr++) {
      const bool rin = t0 + RPW * w + rr < a.T;
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const float xs = has_b ? xv[rr][i][e] + bv[rr][i][e] : xv[rr][i][e];
          xv[rr][i][e] = (rin && i < nv) ? xs : 0.0f;
        }
    }
#pragma unroll
    for (int rr = 0; rr < RPW; rr++) {
      const int row = t0 + RPW * w + rr;
      float s = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; i++)
        if (i < nv)
#pragma unroll
          for (int e = 0; e < 4; e++) s = s + xv[rr][i][e] * xv[rr][i][e];
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, m);
      const float ir = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(s, (float)a.K) + a.neps));
      f4 y = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int i = 0; i < 4; i++)
        if (i < nv && i == qy) {
#pragma unroll
          for (int e = 0; e < 4; e++) y[e] = (xv[rr][i][e] * ir) * (wv[i][e] + a.noff);
          if (row < a.T) {
            const int64_t o = (int64_t)row * a.K + 256 * i + 4 * lane;
            if (a.nb) *reinterpret_cast<f4*>(a.nh + o) = xv[rr][i];
            *reinterpret_cast<f4*>(const_cast<float*>(a.x) + o) = y;
          }
        }
      if (qy == 0 && lane == 0 && row < a.T) a.ninv[row] = ir;
#pragma unroll
      for (int e = 0; e < 4; e++) sx[(RPW * w + rr) * LDX + 4 * lane + e] = y[e];
    }
    // rows NT .. 15 of the LoRA product's token tile: zeros
    for (int i = tid; i < (16 - NT) * LDX; i += 256) sx[NT * LDX + i] = 0.0f;
  }
  __syncthreads();
  float v[NT];
#pragma unroll
  for (int i = 0; i < NT; i++) v[i] = sx[tl * LDX + sg * NT + i];
  // Q8_0 codes: d = amax / 127 over the block (BL adjacent lanes), codes round(x / d)
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < NT; i++) amax = fmaxf(amax, fabsf(v[i]));
#pragma unroll
  for (int m = 1; m < BL; m <<= 1) amax = fmaxf(amax, __shfl_xor(amax, m));
  const float d = __fdiv_rn(amax, 127.0f);
  const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
  _Float16 q[NT];
#pragma unroll
  for (int i = 0; i < NT; i++) q[i] = (_Float16)roundf(__fmul_rn(v[i], id));
  const float dstore = (float)(_Float16)d;
  if (kk < a.Kp) {
    // block elements e0 .. e0 + NT - 1 (e0 = NT qq): half hf = e0 / 16, its k-groups (e0 % 16) / 4 ..
    const int b = kk >> 5, qq = sg % BL, e0 = NT * qq, hf = e0 >> 4, g0 = (e0 & 15) >> 2, kc = b >> 2, j = b & 3;
    u2v* xq = reinterpret_cast<u2v*>(a.xq) + ((((int64_t)(t >> 4) * Kc + kc) * 4 + j) * 64 + (t & 15)) * 2 + hf;
#pragma unroll
    for (int gg = 0; gg < NT / 4; gg++) {
      const half2v lo = {q[4 * gg], q[4 * gg + 1]}, hi = {q[4 * gg + 2], q[4 * gg + 3]};
      u2v wd;
      wd.x = __builtin_bit_cast(uint32_t, lo);
      wd.y = __builtin_bit_cast(uint32_t, hi);
      xq[(g0 + gg) * 16 * 2] = wd;
    }
    const bool real = t < a.T && kk < a.K;
    if (qq == 0) a.xd[((int64_t)kc * a.Tp + t) * 4 + j] = real ? dstore : 0.0f;
    if (a.xdh && qq == 0)
      a.xdh[((int64_t)kc * a.Tp + t) * 4 + j] = real ? __builtin_bit_cast(uint16_t, (_Float16)dstore) : (uint16_t)0;
  }
  if (a.A)  // uniform
    lora_partial_v<NT>(nullptr, mv, a.T, a.A, a.K, a.r, k0, a.K, t0, a.hp, gridDim.y, blockIdx.y, sx, sa, red);
}
extern "C" __global__ __launch_bounds__(256) void rtq_act_prep8_q8_0(ActArgs a) { act_prep_norm<8>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_act_prep4_q8_0(ActArgs a) { act_prep_norm<4>(a); }

// ============================================================== forward GEMM (Q4_0 / Q8_0)
// MFMA orientation: A operand = 16 weight rows x 32 columns, B operand = 32 columns x 16 tokens,
// so output lane l holds token l%16 and weight rows 4(l/16)..4(l/16)+3: one activation scale per
// lane and four consecutive outputs of a y row (one 16-byte store).
// Workgroup = 4 waves sharing one output tile of TT*16 tokens x RG*16 rows; the waves split the
// K range by half chunks (64 columns, two blocks; wave w takes half chunks w, w+4, ...), then
// reduce their partial tiles through LDS.  Each wave keeps its operands in registers in a D-deep
// ring: the loads of item i + D - 1 are issued before item i is computed, all unconditionally
// (clamped indices), so the wait for item i covers only the loads issued D - 1 items earlier.
// Per block: one 16x16x32 f16 MFMA per (token tile, row group) gives the exact integer block
// sums, then acc += isum * (d_w * d_x).
// K-quants: the 6-bit sub-block scales are folded into the weight fragments, so the MFMA
// accumulators sum whole super-blocks exactly (every partial is an integer below 2^24), and the
// f32 epilogue runs once per super-block with the super-block's (d, dmin) and d_x:
//   Q4_K: S1 = sum_j sc_j isum_j (fragment sc_j * u <= 945) and S2 = sum_j m_j bsum_j (fragment
//         m_j: the MFMA sums the activation codes); y += (d d_x) S1 - (dmin d_x) S2;
//   Q6_K: sc = 16 sh + sl (sh in [-8, 7], sl in [0, 15]) so that sh*q and sl*q stay exact f16
//         integers; S = 16 S_hi + S_lo (one rounding, as the integer S converted to f32);
//         y += (d d_x) S.
// Wave w takes super-blocks w, w+4, ... (four half chunks each) instead of half chunks w, w+4.
template <int FMT>
struct WHalf;

template <>
struct WHalf<FMT_Q4_0> {
  u2v q;  // blocks 2h, 2h+1 of the chunk: four code bytes each
  u4v d;  // eight fp16 scales: [j2][i] = row 4g+i, block 2h+j2
  __device__ __forceinline__ void load(const void* wq, const uint16_t* wd, const uint32_t*, int rg, int kc, int h,
                                       int Kc, int lane) {
    q = reinterpret_cast<const u2v*>(wq)[(((uint32_t)rg * Kc + kc) * 64 + lane) * 2 + h];
    d = reinterpret_cast<const u4v*>(wd)[(((uint32_t)rg * Kc + kc) * 2 + h) * 4 + (lane >> 4)];
  }
  __device__ __forceinline__ half8 frag(int j2) const { return q4_0_frag(j2 ? q.y : q.x); }
};

template <>
struct WHalf<FMT_Q8_0> {
  u4v q;  // part h: block 2h in (x, y), block 2h+1 in (z, w)
  u4v d;
  __device__ __forceinline__ void load(const void* wq, const uint16_t* wd, const uint32_t*, int rg, int kc, int h,
                                       int Kc, int lane) {
    q = reinterpret_cast<const u4v*>(wq)[(((uint32_t)rg * Kc + kc) * 2 + h) * 64 + lane];
    d = reinterpret_cast<const u4v*>(wd)[(((uint32_t)rg * Kc + kc) * 2 + h) * 4 + (lane >> 4)];
  }
  __device__ __forceinline__ half8 frag(int j2) const { return j2 ? q8_frag(q.z, q.w) : q8_frag(q.x, q.y); }
};

// sub-block scale word (row lane % 16, blocks 2h, 2h+1) and super-block scales (rows 4g..4g+3)
__device__ __forceinline__ void load_kscales(const uint16_t* wd, const uint32_t* wsb, int rg, int kc, int h, int Kc,
                                             int lane, uint32_t& k, u4v& e) {
  k = reinterpret_cast<const uint32_t*>(wd)[(((uint32_t)rg * Kc + kc) * 16 + (lane & 15)) * 2 + h];
  e = reinterpret_cast<const u4v*>(wsb)[((uint32_t)rg * (Kc >> 1) + (kc >> 1)) * 4 + (lane >> 4)];
}

template <>
struct WHalf<FMT_Q4_K> {
  u2v q;       // unsigned codes, Q4_0 layout
  uint32_t k;  // (sc | m << 8) of block 2h (low half) and 2h+1 (high half), row lane % 16
  u4v e;       // (d | dmin << 16) of rows 4g..4g+3
  __device__ __forceinline__ void load(const void* wq, const uint16_t* wd, const uint32_t* wsb, int rg, int kc, int h,
                                       int Kc, int lane) {
    q = reinterpret_cast<const u2v*>(wq)[(((uint32_t)rg * Kc + kc) * 64 + lane) * 2 + h];
    load_kscales(wd, wsb, rg, kc, h, Kc, lane, k, e);
  }
  // f1 = sc * u (exact, <= 945), f2 = m (every element)
  __device__ __forceinline__ void frags(int j2, half8& f1, half8& f2) const {
    const uint32_t wv = j2 ? (k >> 16) : k;
    const _Float16 sc = (_Float16)(float)(wv & 0x3fu), m = (_Float16)(float)((wv >> 8) & 0x3fu);
    f1 = q4_0_frag<0>(j2 ? q.y : q.x) * sc;
    const half8 mm = {m, m, m, m, m, m, m, m};
    f2 = mm;
  }
};

template <>
struct WHalf<FMT_Q6_K> {
  u4v q;       // int8 codes, Q8_0 layout
  uint32_t k;  // (sc0 | sc1 << 8) of block 2h (low half) and 2h+1 (high half), row lane % 16
  u4v e;       // (d | 0 << 16) of rows 4g..4g+3
  __device__ __forceinline__ void load(const void* wq, const uint16_t* wd, const uint32_t* wsb, int rg, int kc, int h,
                                       int Kc, int lane) {
    q = reinterpret_cast<const u4v*>(wq)[(((uint32_t)rg * Kc + kc) * 2 + h) * 64 + lane];
    load_kscales(wd, wsb, rg, kc, h, Kc, lane, k, e);
  }
  // f1 = sh * q, f2 = sl * q with sc = 16 sh + sl per 16-element sub-block (elements 0..3 of the
  // fragment lie in the block's first sub-block, 4..7 in its second)
  __device__ __forceinline__ void frags(int j2, half8& f1, half8& f2) const {
    const uint32_t wv = j2 ? (k >> 16) : k;
    const int s0 = (int)(int8_t)(wv & 0xffu), s1 = (int)(int8_t)((wv >> 8) & 0xffu);
    const _Float16 h0 = (_Float16)(float)(s0 >> 4), h1 = (_Float16)(float)(s1 >> 4);
    const _Float16 l0 = (_Float16)(float)(s0 & 15), l1 = (_Float16)(float)(s1 & 15);
    const half8 qf = j2 ? q8_frag(q.z, q.w) : q8_frag(q.x, q.y);
    const half8 sh = {h0, h0, h0, h0, h1, h1, h1, h1}, sl = {l0, l0, l0, l0, l1, l1, l1, l1};
    f1 = qf * sh;
    f2 = qf * sl;
  }
};

// scale i (0..3) of block j2 from the 16-byte scale vector: fp16 number 4*j2 + i
__device__ __forceinline__ float wscale(const u4v& d, int j2, int i) {
  const uint32_t w = comp(d, 2 * j2 + (i >> 1));
  return h2f((uint16_t)((i & 1) ? (w >> 16) : (w & 0xffffu)));
}

template <int FMT, int TT, int RG>
struct FwdSlot {
  WHalf<FMT> w[RG];
  u4v x[TT][2];  // activation fragments of blocks 2h, 2h+1
  float xs[TT][2];
};


template <int FMT, int TT, int RG, int D, bool DBG, int NW = 4>
__device__ __forceinline__ void fwd_tile(const FwdArgs& a) {
  constexpr bool KQ = is_kquant(FMT);
  static_assert(NW == 4 || (NW == 8 && !KQ), "K-quant tiles split K over four waves");
  __shared__ f4 red[4][TT * RG][64];
  __shared__ float sh[TT * 16][RTQ_LDS_RANK + 1];  // LoRA down projection rows of this tile's tokens
  __shared__ float sb[RG * 16][RTQ_LDS_RANK + 1];  // LoRA B rows of this tile
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, li = lane & 15, g = lane >> 4;
  const int Kc = a.Kp / 128;
  const int ngroups = a.Np / 16, ntt = a.Tp / 16;
  const int rg0 = blockIdx.x * RG, tt0 = blockIdx.y * TT;
  const int hc0 = blockIdx.z * a.kc_per_split * 2;
  const int hc1 = min(hc0 + a.kc_per_split * 2, 2 * Kc);
  // items (half chunks) of this wave; K-quant splits hold whole super-blocks (four half chunks)
  int nit;
  if (KQ) {
    const int nsb = (hc1 - hc0) >> 2;
    nit = nsb > w ? (nsb - w + 3) / 4 * 4 : 0;
  } else {
    nit = hc1 - hc0 > w ? (hc1 - hc0 - w + NW - 1) / NW : 0;
  }
  auto item_hc = [&](int it) { return KQ ? hc0 + 4 * (w + 4 * (it >> 2)) + (it & 3) : hc0 + w + NW * it; };
  const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  f4 acc[TT][RG];
  f4 s1[KQ ? TT : 1][KQ ? RG : 1], s2[KQ ? TT : 1][KQ ? RG : 1];  // K-quant super-block sums
#pragma unroll
  for (int i = 0; i < TT; i++)
#pragma unroll
    for (int r = 0; r < RG; r++) acc[i][r] = zero;
  if (KQ) {
#pragma unroll
    for (int i = 0; i < (KQ ? TT : 1); i++)
#pragma unroll
      for (int r = 0; r < (KQ ? RG : 1); r++) s1[i][r] = s2[i][r] = zero;
  }

  const u4v* XQ = reinterpret_cast<const u4v*>(a.xq);
  const float2* XD = reinterpret_cast<const float2*>(a.xd);
  int rgc[RG], ttc[TT];
#pragma unroll
  for (int r = 0; r < RG; r++) rgc[r] = min(rg0 + r, ngroups - 1);
#pragma unroll
  for (int i = 0; i < TT; i++) ttc[i] = min(tt0 + i, ntt - 1);
  FwdSlot<FMT, TT, RG> sl[D];
  const bool lead = blockIdx.z == 0;
  const bool lora = a.hp && lead;
  // the up-projection of row group rg reads the ranks of its member of a block-diagonal adapter
  // only (the other B entries are zeros); the tile's rank span is staged in LDS when it fits
  int span0 = 0, span1 = 0;
  if (lora) rb_span(a.rb, a.r, rg0 * 16, min((rg0 + RG) * 16, a.N), span0, span1);
  const bool lora_lds = lora && span1 - span0 <= RTQ_LDS_RANK;

  auto issue = [&](FwdSlot<FMT, TT, RG>& S, int it) {
    const int hc = min(item_hc(min(it, max(nit - 1, 0))), 2 * Kc - 1);  // clamped: always a valid half chunk
    const int kc = hc >> 1, h = hc & 1;
#pragma unroll
    for (int r = 0; r < RG; r++) S.w[r].load(a.wq, a.wd, a.wsb, rgc[r], kc, h, Kc, lane);
#pragma unroll
    for (int i = 0; i < TT; i++) {
      const uint32_t base = (((uint32_t)ttc[i] * Kc + kc) * 4 + 2 * h) * 64 + lane;
      S.x[i][0] = XQ[base];
      S.x[i][1] = XQ[base + 64];
      const float2 s2 = XD[((uint32_t)kc * a.Tp + ttc[i] * 16 + li) * 2 + h];
      S.xs[i][0] = s2.x;
      S.xs[i][1] = s2.y;
    }
  };
  auto compute = [&](const FwdSlot<FMT, TT, RG>& S, int it) {
    const int hc = item_hc(it);
    if constexpr (KQ) {
#pragma unroll
      for (int j2 = 0; j2 < 2; j2++) {
        half8 f1[RG], f2[RG];
#pragma unroll
        for (int r = 0; r < RG; r++) S.w[r].frags(j2, f1[r], f2[r]);
#pragma unroll
        for (int i = 0; i < TT; i++) {
          const half8 xf = __builtin_bit_cast(half8, S.x[i][j2]);
#pragma unroll
          for (int r = 0; r < RG; r++) {
            s1[i][r] = mfma_f16(f1[r], xf, s1[i][r]);
            s2[i][r] = mfma_f16(f2[r], xf, s2[i][r]);
          }
        }
      }
      if ((it & 3) == 3) {  // last half chunk of the super-block: f32 epilogue, then restart the sums
        const int sb = hc >> 2, nsb = a.K / 256;
#pragma unroll
        for (int i = 0; i < TT; i++) {
          const float xs = S.xs[i][0];  // the super-block's Q8_K d of token li
#pragma unroll
          for (int r = 0; r < RG; r++) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
              const uint32_t ev = comp(S.w[r].e, e);
              const float dd = h2f((uint16_t)(ev & 0xffffu)) * xs;
              if (FMT == FMT_Q4_K) {
                const float dm = h2f((uint16_t)(ev >> 16)) * xs;
                acc[i][r][e] = fmaf(dd, s1[i][r][e], fmaf(-dm, s2[i][r][e], acc[i][r][e]));
              } else {
                acc[i][r][e] = fmaf(dd, fmaf(16.0f, s1[i][r][e], s2[i][r][e]), acc[i][r][e]);
              }
              if (DBG) {
                const int t = (tt0 + i) * 16 + li, n = (rg0 + r) * 16 + 4 * g + e;
                if (t < a.T && n < a.N && sb < nsb) {
                  if (FMT == FMT_Q4_K) {
                    a.isums[(((int64_t)t * a.N + n) * nsb + sb) * 2] = (int32_t)s1[i][r][e];
                    a.isums[(((int64_t)t * a.N + n) * nsb + sb) * 2 + 1] = (int32_t)s2[i][r][e];
                  } else {
                    a.isums[((int64_t)t * a.N + n) * nsb + sb] = 16 * (int32_t)s1[i][r][e] + (int32_t)s2[i][r][e];
                  }
                }
              }
            }
            s1[i][r] = zero;
            s2[i][r] = zero;
          }
        }
      }
    } else {
#pragma unroll
      for (int j2 = 0; j2 < 2; j2++) {
        half8 wf[RG];
        float sc[RG][4];
#pragma unroll
        for (int r = 0; r < RG; r++) {
          wf[r] = S.w[r].frag(j2);
#pragma unroll
          for (int i = 0; i < 4; i++) sc[r][i] = wscale(S.w[r].d, j2, i);
        }
#pragma unroll
        for (int i = 0; i < TT; i++) {
          const half8 xf = __builtin_bit_cast(half8, S.x[i][j2]);
          const float xs = S.xs[i][j2];
#pragma unroll
          for (int r = 0; r < RG; r++) {
            const f4 c = mfma_f16(wf[r], xf, zero);
            if (DBG) {
              const int t = (tt0 + i) * 16 + li, b = hc * 2 + j2, nb = a.K / 32;
#pragma unroll
              for (int e = 0; e < 4; e++) {
                const int n = (rg0 + r) * 16 + 4 * g + e;
                if (t < a.T && n < a.N && b < nb) a.isums[((int64_t)t * a.N + n) * nb + b] = (int32_t)c[e];
              }
            }
#pragma unroll
            for (int e = 0; e < 4; e++) acc[i][r][e] = fmaf(c[e], sc[r][e] * xs, acc[i][r][e]);
          }
        }
      }
    }
  };
  // D-deep ring; item it lives in slot it % D
#pragma unroll
  for (int s = 0; s < D - 1; s++) issue(sl[s], s);
  if (lora_lds && threadIdx.x < 256) {
    // stage h rows of this tile's tokens and B rows of its weight rows, 16 ranks at a time, by the
    // first four waves; the loads are issued after the ring prologue and overlap it
    for (int j0 = span0; j0 < span1; j0 += 16) {  // staged rank j at column j - span0
      constexpr int NH = TT * 16 * 16 / 256, NB = (RG * 16 * 16 + 255) / 256;
      float hv[NH], bv[NB];
#pragma unroll
      for (int k = 0; k < NH; k++) {
        const int e = threadIdx.x + 256 * k, tl = e >> 4, j = j0 + (e & 15);
        hv[k] = sum_partials(a.hp, (int64_t)min(tt0 * 16 + tl, a.T - 1) * a.r + min(j, a.r - 1), a.nhp);
      }
#pragma unroll
      for (int k = 0; k < NB; k++) {
        const int e = min(threadIdx.x + 256 * k, RG * 256 - 1), nl = e >> 4, j = j0 + (e & 15);
        bv[k] = a.lb[(int64_t)min(rg0 * 16 + nl, a.N - 1) * a.r + min(j, a.r - 1)];
      }
#pragma unroll
      for (int k = 0; k < NH; k++) {
        const int e = threadIdx.x + 256 * k;
        sh[e >> 4][j0 - span0 + (e & 15)] = hv[k];
      }
#pragma unroll
      for (int k = 0; k < NB; k++) {
        const int e = threadIdx.x + 256 * k;
        if (e < RG * 256) sb[e >> 4][j0 - span0 + (e & 15)] = bv[k];
      }
    }
  }
  for (int it0 = 0; it0 < nit; it0 += D) {
#pragma unroll
    for (int s = 0; s < D; s++) {
      issue(sl[(s + D - 1) % D], it0 + s + D - 1);
      __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of this item's math
      if (it0 + s < nit) compute(sl[s], it0 + s);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // ---- reduce the waves' partial tiles (eight waves: w + 4 into w first), then wave w < 4
  // finalises pairs p = w, w + 4, ...
  if (NW == 8) {
    if (w >= 4) {
#pragma unroll
      for (int i = 0; i < TT; i++)
#pragma unroll
        for (int r = 0; r < RG; r++) red[w - 4][i * RG + r][lane] = acc[i][r];
    }
    __syncthreads();
    if (w < 4) {
#pragma unroll
      for (int i = 0; i < TT; i++)
#pragma unroll
        for (int r = 0; r < RG; r++) acc[i][r] += red[w][i * RG + r][lane];
    }
    __syncthreads();
  }
  if (w < 4) {
#pragma unroll
    for (int i = 0; i < TT; i++)
#pragma unroll
      for (int r = 0; r < RG; r++) red[w][i * RG + r][lane] = acc[i][r];
  }
  __syncthreads();
  const bool split = gridDim.z > 1;
  for (int p = w; p < (w < 4 ? TT * RG : 0); p += 4) {
    const int i = p / RG, r = p % RG;
    const f4 v0 = red[0][p][lane], v1 = red[1][p][lane], v2 = red[2][p][lane], v3 = red[3][p][lane];
    f4 v;
#pragma unroll
    for (int e = 0; e < 4; e++) v[e] = (v0[e] + v1[e]) + (v2[e] + v3[e]);
    const int t = (tt0 + i) * 16 + li;
    const int nb0 = (rg0 + r) * 16;
    const int n0 = nb0 + 4 * g;
    if (nb0 >= a.N) continue;  // whole row group is padding (uniform over the wave)
    // LoRA up: lacc[e] = sum_j B[n0+e][j] h[t][j]  (f32 MFMA, A operand = B rows, B operand = h rows)
    f4 lacc = zero;
    int lo = 0, hi = 0;  // this row group's ranks
    if (lora) rb_span(a.rb, a.r, nb0, nb0 + 16, lo, hi);
    if (lora_lds) {
      for (int j0 = lo; j0 < hi; j0 += 4) {
        const int j = j0 + g, jc = min(j, hi - 1) - span0;
        const float hv = sh[i * 16 + li][jc], bv = sb[r * 16 + li][jc];
        lacc = mfma_f32((nb0 + li < a.N && j < hi) ? bv : 0.0f, (t < a.T && j < hi) ? hv : 0.0f, lacc);
      }
    } else if (lora) {  // rank span above the LDS staging limit: straight from global memory
      const int tc = min(t, a.T - 1);
      const int nrow = min(nb0 + li, a.N - 1);
      for (int j0 = lo; j0 < hi; j0 += 4) {
        const int j = j0 + g, jc = min(j, hi - 1);
        const float hv = sum_partials(a.hp, (int64_t)tc * a.r + jc, a.nhp);
        const float bv = a.lb[(int64_t)nrow * a.r + jc];
        lacc = mfma_f32((nb0 + li < a.N && j < hi) ? bv : 0.0f, (t < a.T && j < hi) ? hv : 0.0f, lacc);
      }
    }
    if (t < a.T) {
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int n = n0 + e;
        float o = v[e];
        if (a.bias && lead) o = o + a.bias[min(n, a.N - 1)];
        if (lora) o = o + a.s * lacc[e];
        v[e] = o;
      }
      float* yr = a.y + (int64_t)t * a.N;
      if (split) {
#pragma unroll
        for (int e = 0; e < 4; e++)
          if (n0 + e < a.N) atomicAdd(&yr[n0 + e], v[e]);
      } else if ((a.N & 3) == 0 && n0 + 3 < a.N) {
        *reinterpret_cast<f4*>(yr + n0) = v;
      } else {
#pragma unroll
        for (int e = 0; e < 4; e++)
          if (n0 + e < a.N) yr[n0 + e] = v[e];
      }
    }
  }
}

// wide: 4 token tiles x 3 row groups per workgroup (64 x 48 outputs), 2-deep ring;
// skinny (T <= 16): 1 token tile x 4 row groups, 4-deep ring, split K across workgroups too.
#define RTQ_FWD(NAME, FMT, TT, RG, D, DBG)                                   \
  extern "C" __global__ __launch_bounds__(256) void NAME(FwdArgs a) {        \
    fwd_tile<FMT, TT, RG, D, DBG>(a);                                        \
  }
RTQ_FWD(rtq_fwd_q4_0_w, FMT_Q4_0, 4, 3, 2, false)
// eight waves splitting K (two per SIMD), Q4_0 / Q8_0
#define RTQ_FWD8(NAME, FMT, TT, RG, D)                                       \
  extern "C" __global__ __launch_bounds__(512) void NAME(FwdArgs a) {        \
    fwd_tile<FMT, TT, RG, D, false, 8>(a);                                   \
  }
RTQ_FWD8(rtq_fwd_q4_0_w8, FMT_Q4_0, 4, 3, 2)
RTQ_FWD8(rtq_fwd_q8_0_w8, FMT_Q8_0, 4, 3, 2)
// 64 tokens x 32 rows: where 48-row tiles would leave CUs without a workgroup (thin outputs)
RTQ_FWD8(rtq_fwd_q4_0_w8r2, FMT_Q4_0, 4, 2, 2)
RTQ_FWD8(rtq_fwd_q8_0_w8r2, FMT_Q8_0, 4, 2, 2)
// 64 tokens x 16 rows: where 32-row tiles would still leave CUs without a workgroup
RTQ_FWD8(rtq_fwd_q4_0_w8r1, FMT_Q4_0, 4, 1, 2)
RTQ_FWD8(rtq_fwd_q8_0_w8r1, FMT_Q8_0, 4, 1, 2)
RTQ_FWD(rtq_fwd_q4_0_s, FMT_Q4_0, 1, 4, 4, false)
RTQ_FWD(rtq_fwd_q8_0_w, FMT_Q8_0, 4, 3, 2, false)
RTQ_FWD(rtq_fwd_q8_0_s, FMT_Q8_0, 1, 4, 4, false)
RTQ_FWD(rtq_fwd_q4_0_w_isums, FMT_Q4_0, 4, 3, 2, true)
RTQ_FWD(rtq_fwd_q4_0_s_isums, FMT_Q4_0, 1, 4, 4, true)
RTQ_FWD(rtq_fwd_q8_0_w_isums, FMT_Q8_0, 4, 3, 2, true)
RTQ_FWD(rtq_fwd_q8_0_s_isums, FMT_Q8_0, 1, 4, 4, true)
RTQ_FWD(rtq_fwd_q4_k_w, FMT_Q4_K, 4, 2, 2, false)
RTQ_FWD(rtq_fwd_q4_k_s, FMT_Q4_K, 1, 4, 4, false)
RTQ_FWD(rtq_fwd_q6_k_w, FMT_Q6_K, 4, 2, 2, false)
RTQ_FWD(rtq_fwd_q6_k_s, FMT_Q6_K, 1, 4, 4, false)
RTQ_FWD(rtq_fwd_q4_k_w_isums, FMT_Q4_K, 4, 2, 2, true)
RTQ_FWD(rtq_fwd_q4_k_s_isums, FMT_Q4_K, 1, 4, 4, true)
RTQ_FWD(rtq_fwd_q6_k_w_isums, FMT_Q6_K, 4, 2, 2, true)
RTQ_FWD(rtq_fwd_q6_k_s_isums, FMT_Q6_K, 1, 4, 4, true)

// ============================================================== forward GEMM, large grids (Q4_0 / Q8_0)
// For outputs of at least a workgroup per CU in 128 x 128 tiles (128 x 64: rtq_mm64_*, 128 x 32:
// rtq_mm32_*).  Workgroup = 4 waves, tile 128 weight rows (8 row groups) x 16 TTN tokens (TTN = 8,
// 4 or 2 token tiles); wave w computes row groups 2w, 2w+1 x all TTN token tiles: a weight
// fragment is unpacked once per TTN token tiles, the activation fragments are shared by the four
// waves through LDS.  Per half chunk (64 columns, two blocks) the workgroup's operands - weight
// codes and scales, activation codes and scales - are copied global -> LDS by buffer loads with an
// LDS destination (no VGPR staging) into a RING-stage ring: while stage s is computed, the loads
// of stages s + 1 .. s + RING - 2 are in flight.  One barrier per stage; the wait before it names
// the loads of stage s only (the raw s_barrier keeps the compiler from draining every load there).
// The kernel is bound by issue and latency more than by either pipe (128 x 64 tiles at the
// Qwen3-0.6B q|k|v shape, 512 tokens: one workgroup per CU, VALU busy ~25 %, MFMA ~10 %): 32-token tiles, at
// two or three workgroups per CU, beat them there, while a deeper ring (6) and eight waves per
// workgroup did not.  The 1D grid deals the tiles, ordered token block
// by token block, to the eight XCDs in contiguous ranges: the workgroups running on one XCD share
// one token block's activations in that XCD's L2 while they stream weight rows.  Arithmetic as
// fwd_tile: exact integer block sums from the f16 MFMA, acc += isum * (d_w * d_x), with the scale
// products formed by a 4-block f16 MFMA in the layout of the block-sum tiles.
#define RTQ_LDSP(p) ((__attribute__((address_space(3))) void*)(p))

template <int FMT, int TTN>
struct MmStage {  // one half chunk in LDS, in 16-byte units; TTN token tiles of 16 per workgroup
  static constexpr int XQ = 0;                                       // [tt TTN][j2 2][lane 64] codes
  static constexpr int WQ = TTN * 2 * 64;                            // [rg 8][lane 64] Q4_0 8 B, Q8_0 16 B
  static constexpr int WD = WQ + (FMT == FMT_Q4_0 ? 8 * 64 / 2 : 8 * 64);  // [rg 8][row 16] fp16 scale pairs
  static constexpr int XD = WD + 8 * 4;                              // [t 16 TTN] fp16 activation scale pairs
  static constexpr int NXD = TTN >= 4 ? TTN / 4 : 1;                 // loads of activation scales (64 tokens each)
  static constexpr int SIZE = XD + 16 * NXD;                         // (TTN 2: the load's last 32 tokens unused)
  static constexpr int NX = 2 * TTN;                                 // loads of activation fragments
  static constexpr int NWQ = FMT == FMT_Q4_0 ? 16 : 8;               // loads of weight codes
  static constexpr int LOADS = NX + NWQ + 2 + NXD;                   // wave-wide loads per stage
};

// s_waitcnt immediate: vmcnt <= n (0..63; low four bits, then bits 15:14), expcnt and lgkmcnt free
constexpr int vm_wait_imm(int n) { return 0x0F70 | (n & 15) | (((n >> 4) & 3) << 14); }

// wait until at most after * L vector-memory loads of this wave are outstanding (after: 0 .. 6)
template <int L>
__device__ __forceinline__ void vm_wait_stages(int after) {
  switch (after) {
    case 0: __builtin_amdgcn_s_waitcnt(vm_wait_imm(0)); break;
    case 1: __builtin_amdgcn_s_waitcnt(vm_wait_imm(L)); break;
    case 2: __builtin_amdgcn_s_waitcnt(vm_wait_imm(2 * L)); break;
    case 3: __builtin_amdgcn_s_waitcnt(vm_wait_imm(3 * L)); break;
    case 4: __builtin_amdgcn_s_waitcnt(vm_wait_imm(4 * L)); break;
    case 5: __builtin_amdgcn_s_waitcnt(vm_wait_imm(5 * L)); break;
    default: __builtin_amdgcn_s_waitcnt(vm_wait_imm(6 * L)); break;
  }
}

template <int FMT, int TTN, int RING>
__device__ __forceinline__ void mm_tile(const FwdArgs& a) {
  using St = MmStage<FMT, TTN>;
  extern __shared__ u4v mm_lds[];
  const int lane = threadIdx.x & 63, li = lane & 15, g = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int Kc = a.Kp / 128, nhc = a.Kp / 64;
  const int ngroups = a.Np / 16, ntt = a.Tp / 16;
  // XCD-aware tile order: workgroup id -> (XCD id % 8, slot id / 8) -> a contiguous range of the
  // tile order per XCD.  The order takes the row blocks in groups of MM_GR: within a group token
  // block by token block, the group's row blocks of one token block consecutive.  The ~64
  // workgroups an XCD runs at once then cover MM_GR row blocks x 64 / MM_GR token blocks, whose
  // weight rows and activation columns they share in that XCD's L2 (row blocks fastest over all
  // token blocks would re-read every weight row from HBM once per token block).
  constexpr int MM_GR = 8;
  const int nrb = (ngroups + 7) / 8, ntb = ntt / TTN, ntiles = nrb * ntb;
  const int id = blockIdx.x, xcd = id & 7, per = ntiles >> 3, rem = ntiles & 7;
  const int q = xcd * per + min(xcd, rem) + (id >> 3);
  const int gfull = nrb / MM_GR, q0 = gfull * MM_GR * ntb;
  int rb, tb;
  if (q < q0) {
    const int in = q % (MM_GR * ntb);
    rb = (q / (MM_GR * ntb)) * MM_GR + in % MM_GR;
    tb = in / MM_GR;
  } else {  // the last, partial group of nrb % MM_GR row blocks
    const int gr = nrb - gfull * MM_GR, in = q - q0;
    rb = gfull * MM_GR + in % gr;
    tb = in / gr;
  }
  const int rg0 = rb * 8, tt0 = tb * TTN;

  // Operands reach LDS by buffer loads with the LDS destination (4 or 16 bytes per lane; gfx950
  // has no 8-byte form, so 8-byte items - Q4_0 half-chunk codes, scale pairs - go as pairs of
  // words).  Every lane's byte offset for half chunk 0 is computed once; a half chunk adds a
  // wave-uniform offset (kc * A + h * B per operand) in an SGPR.  The buffer ranges are the arrays'
  // sizes, so a load past an array's end reads zeros instead of faulting.
  const uint32_t nb_x = (uint32_t)a.Tp * a.Kp * 2, nb_xd = (uint32_t)Kc * a.Tp * 8;
  const uint32_t nb_w = (uint32_t)a.Np * a.Kp / (FMT == FMT_Q4_0 ? 2 : 1), nb_wd = (uint32_t)a.Np * a.Kp / 16;
  const __amdgpu_buffer_rsrc_t rs_x = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(a.xq), (short)0, nb_x, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs_xd = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.xdh), (short)0, nb_xd, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs_w = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(a.wq), (short)0, nb_w, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs_wd = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.wdr), (short)0, nb_wd, 0x00020000);
  // Every wave issues the same kinds of loads (no per-wave branching in the loop): KX activation
  // fragments (i = w + 4k), KW weight-code loads (iw = w + 4k), and one scale load: waves 0, 1 a
  // weight scale-pair word row, waves 2 .. 1 + NXD the activation scales (NXD is 1 or 2).
  constexpr int KX = St::NX / 4, KW = St::NWQ / 4;
  static_assert(St::NX % 4 == 0 && St::NWQ % 4 == 0 && St::NXD <= 2, "load split over four waves");
  uint32_t vx[KX], vw[KW], ve = 0;
#pragma unroll
  for (int k = 0; k < KX; k++) {  // activation fragments: token tile i / 2, block 2h + i % 2
    const int i = w + 4 * k;
    const uint32_t ttg = (uint32_t)min(tt0 + (i >> 1), ntt - 1);
    vx[k] = ((ttg * Kc * 4 + (i & 1)) * 64 + lane) * 16;
  }
#pragma unroll
  for (int k = 0; k < KW; k++) {  // weight codes
    const int iw = w + 4 * k;
    if (FMT == FMT_Q4_0) {  // row group iw / 2, words 64 m .. 64 m + 63 of its 128
      const int wi = (iw & 1) * 64 + lane;
      const uint32_t rgg = (uint32_t)min(rg0 + (iw >> 1), ngroups - 1);
      vw[k] = ((rgg * Kc * 64 + (wi >> 1)) * 4 + (wi & 1)) * 4;
    } else {
      const uint32_t rgg = (uint32_t)min(rg0 + iw, ngroups - 1);
      vw[k] = (rgg * Kc * 2 * 64 + lane) * 16;
    }
  }
  if (w < 2) {  // weight scale pairs: word wi -> row wi % 16 of row group wi / 16
    const int wi = w * 64 + lane;
    const uint32_t rgg = (uint32_t)min(rg0 + (wi >> 4), ngroups - 1);
    ve = ((rgg * Kc * 16 + (wi & 15)) * 2) * 4;
  } else if (w - 2 < St::NXD) {  // fp16 activation scales of blocks 2h, 2h+1: word wi -> token wi
    const int wi = (w - 2) * 64 + lane;
    ve = (uint32_t)min(tt0 * 16 + wi, a.Tp - 1) * 8;
  }
  auto issue = [&](int st, int hc) {
    u4v* S = mm_lds + st * St::SIZE;
    const uint32_t kc = hc >> 1, h = hc & 1;
#pragma unroll
    for (int k = 0; k < KX; k++)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_x, RTQ_LDSP(S + St::XQ + (w + 4 * k) * 64), 16, vx[k], hc * 2048u, 0, 0);
#pragma unroll
    for (int k = 0; k < KW; k++) {
      const int iw = w + 4 * k;
      if (FMT == FMT_Q4_0)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_w, RTQ_LDSP(S + St::WQ + (iw >> 1) * 32 + (iw & 1) * 16), 4, vw[k],
                                                 kc * 1024u + h * 8u, 0, 0);
      else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_w, RTQ_LDSP(S + St::WQ + iw * 64), 16, vw[k], hc * 1024u, 0, 0);
    }
    if (w < 2)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_wd, RTQ_LDSP(S + St::WD + w * 16), 4, ve, kc * 128u + h * 4u, 0, 0);
    else if (w - 2 < St::NXD)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_xd, RTQ_LDSP(S + St::XD + (w - 2) * 16), 4, ve,
                                               kc * (uint32_t)a.Tp * 8u + h * 4u, 0, 0);
  };

  const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  const f16v zero16 = {};
  f4 acc[TTN][2];  // [token tile][row group]
#pragma unroll
  for (int i = 0; i < TTN; i++)
#pragma unroll
    for (int r = 0; r < 2; r++) acc[i][r] = zero;

  // Per token tile, one 4-block f16 MFMA (16x16x4, k slot 0 only) forms the scale products
  // d_w[row] * d_x[token] of block b = (row group r, block j2) = (b >> 1, b & 1) - exact in f32,
  // fp16 times fp16 - in the layout of the block-sum tiles, so the epilogue is one FMA per output
  // element and block.
  auto compute = [&](int st) {
    const u4v* S = mm_lds + st * St::SIZE;
    half8 wf[2][2];  // [row group][block]
#pragma unroll
    for (int r = 0; r < 2; r++) {
      const int rl = 2 * w + r;
      if (FMT == FMT_Q4_0) {
        const u2v q2 = reinterpret_cast<const u2v*>(S + St::WQ)[rl * 64 + lane];
        wf[r][0] = q4_0_frag(q2.x);
        wf[r][1] = q4_0_frag(q2.y);
      } else {
        const u4v qv = S[St::WQ + rl * 64 + lane];
        wf[r][0] = q8_frag(qv.x, qv.y);
        wf[r][1] = q8_frag(qv.z, qv.w);
      }
    }
    // scale MFMA operands: lane group g = 2 r + j2 holds row li of row group 2w + r, block j2
    const uint32_t dwp = reinterpret_cast<const uint32_t*>(S + St::WD)[(2 * w + (g >> 1)) * 16 + li];
    const u2v dwa = {(g & 1) ? (dwp >> 16) : (dwp & 0xffffu), 0u};
    const half4 sa = __builtin_bit_cast(half4, dwa);
    f16v sc[2];
    f4 c[2][2][2];  // [pipeline slot][row group][block]
    auto products = [&](int i, int b) {
      const uint32_t xsv = reinterpret_cast<const uint32_t*>(S + St::XD)[i * 16 + li];
      const u2v xsa = {(g & 1) ? (xsv >> 16) : (xsv & 0xffffu), 0u};
      sc[b] = __builtin_amdgcn_mfma_f32_16x16x4f16(sa, __builtin_bit_cast(half4, xsa), zero16, 0, 0, 0);
#pragma unroll
      for (int j2 = 0; j2 < 2; j2++) {
        const half8 xf = __builtin_bit_cast(half8, S[St::XQ + (i * 2 + j2) * 64 + lane]);
#pragma unroll
        for (int r = 0; r < 2; r++) c[b][r][j2] = mfma_f16(wf[r][j2], xf, zero);
      }
    };
    // software pipeline over the token tiles: the MFMAs of tile i + 1 are issued before the FMAs
    // that consume tile i
    products(0, 0);
#pragma unroll
    for (int i = 0; i < TTN; i++) {
      if (i + 1 < TTN) products(i + 1, (i + 1) & 1);
#pragma unroll
      for (int r = 0; r < 2; r++)
#pragma unroll
        for (int j2 = 0; j2 < 2; j2++)
#pragma unroll
          for (int e = 0; e < 4; e++)
            acc[i][r][e] = fmaf(c[i & 1][r][j2][e], sc[i & 1][4 * (2 * r + j2) + e], acc[i][r][e]);
    }
  };

  // RING-stage ring over half chunks: stages s + 1 .. s + RING - 2 are in flight while stage s is
  // computed.  Each wave issues at least MINL loads per stage, so "at most MINL x (stages issued
  // after s) outstanding" at the top of step s means stage s has landed.  The loop is unrolled by
  // the ring size so that every stage's LDS offsets are immediates.
  static_assert(RING >= 3 && (RING - 2) * (KX + KW + 2) <= 63, "ring depth within the load counter");
  constexpr int MINL = KX + KW + (St::NXD >= 2 ? 1 : 0);
#pragma unroll
  for (int s = 0; s < RING - 1; s++)
    if (s < nhc) issue(s, s);
  for (int hc0 = 0; hc0 < nhc; hc0 += RING) {
#pragma unroll
    for (int u = 0; u < RING; u++) {
      const int hc = hc0 + u;
      if (hc < nhc) {
        vm_wait_stages<MINL>(min(RING - 2, nhc - 1 - hc));
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (hc + RING - 1 < nhc) issue((u + RING - 1) % RING, hc + RING - 1);
        compute(u);
      }
    }
  }

  // ---- epilogue: bias, LoRA up-projection, y.  The up-projection reads, per row group, only the
  // ranks of its member of a block-diagonal adapter (the other B entries are zeros); h and B rows of
  // the tile's rank span are staged in LDS over the ring, RTQ_LDS_RANK ranks at a time.
  const bool lora = a.hp != nullptr;
  float(*sh)[RTQ_LDS_RANK + 1] = reinterpret_cast<float(*)[RTQ_LDS_RANK + 1]>(mm_lds);
  float(*sb)[RTQ_LDS_RANK + 1] = sh + 16 * TTN;
  int span0 = 0, span1 = 0;  // ranks read by the tile's rows (workgroup-uniform)
  int win0[2] = {0, 0}, win1[2] = {0, 0};  // ranks read by row group 2w + r (wave-uniform)
  if (lora) {
    rb_span(a.rb, a.r, rg0 * 16, min(rg0 * 16 + 128, a.N), span0, span1);
#pragma unroll
    for (int r = 0; r < 2; r++) rb_span(a.rb, a.r, (rg0 + 2 * w + r) * 16, (rg0 + 2 * w + r) * 16 + 16, win0[r], win1[r]);
  }
  f4 lacc[TTN][2];
#pragma unroll
  for (int i = 0; i < TTN; i++)
#pragma unroll
    for (int r = 0; r < 2; r++) lacc[i][r] = zero;
  for (int c0 = span0; c0 < span1; c0 += RTQ_LDS_RANK) {
    const int c1 = min(c0 + RTQ_LDS_RANK, span1);
    __builtin_amdgcn_s_barrier();  // every wave is past its last read of the ring / previous chunk
    asm volatile("" ::: "memory");
    for (int j0 = c0; j0 < c1; j0 += 16) {
      float hv[8], bv[8];
#pragma unroll
      for (int k = 0; k < 8; k++) {  // rows e / 16: 16 TTN token rows of h, 128 weight rows of B
        const int e = threadIdx.x + 256 * k, tl = e >> 4, j = min(j0 + (e & 15), a.r - 1);
        hv[k] = tl < 16 * TTN ? sum_partials(a.hp, (int64_t)min(tt0 * 16 + tl, a.T - 1) * a.r + j, a.nhp) : 0.0f;
        bv[k] = a.lb[(int64_t)min(rg0 * 16 + tl, a.N - 1) * a.r + j];
      }
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const int e = threadIdx.x + 256 * k, jl = j0 - c0 + (e & 15);
        if ((e >> 4) < 16 * TTN) sh[e >> 4][jl] = hv[k];
        sb[e >> 4][jl] = bv[k];
      }
    }
    __syncthreads();
    // lacc[e] += sum_j B[n0+e][j] h[t][j] over this chunk's part of the row group's window (f32
    // MFMA, A operand = B rows, B operand = h rows; lane group g takes rank j0 + g)
#pragma unroll
    for (int r = 0; r < 2; r++) {
      const int lo = max(win0[r], c0), hi = min(win1[r], c1);
      const int nb0 = (rg0 + 2 * w + r) * 16, rl = (2 * w + r) * 16;
      for (int j0 = lo; j0 < hi; j0 += 4) {
        const int j = j0 + g, jl = min(j, hi - 1) - c0;
        const float bv = (nb0 + li < a.N && j < hi) ? sb[rl + li][jl] : 0.0f;
#pragma unroll
        for (int i = 0; i < TTN; i++) {
          const float hv = (tt0 * 16 + i * 16 + li < a.T && j < hi) ? sh[i * 16 + li][jl] : 0.0f;
          lacc[i][r] = mfma_f32(bv, hv, lacc[i][r]);
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < TTN; i++) {
#pragma unroll
    for (int r = 0; r < 2; r++) {
      const int t = tt0 * 16 + i * 16 + li;
      const int nb0 = (rg0 + 2 * w + r) * 16, n0 = nb0 + 4 * g;
      if (nb0 >= a.N) continue;  // whole row group is padding (uniform over the wave)
      if (t < a.T) {
        f4 v = acc[i][r];
#pragma unroll
        for (int e = 0; e < 4; e++) {
          float o = v[e];
          if (a.bias) o = o + a.bias[min(n0 + e, a.N - 1)];
          if (lora) o = o + a.s * lacc[i][r][e];
          v[e] = o;
        }
        float* yr = a.y + (int64_t)t * a.N;
        if ((a.N & 3) == 0 && n0 + 3 < a.N) {
          *reinterpret_cast<f4*>(yr + n0) = v;
        } else {
#pragma unroll
          for (int e = 0; e < 4; e++)
            if (n0 + e < a.N) yr[n0 + e] = v[e];
        }
      }
    }
  }
}

extern "C" __global__ __launch_bounds__(256) void rtq_mm_q4_0(FwdArgs a) { mm_tile<FMT_Q4_0, 8, RTQ_MM_RING>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_mm_q8_0(FwdArgs a) { mm_tile<FMT_Q8_0, 8, RTQ_MM_RING>(a); }
// 128 rows x 64 tokens: twice the grid, for outputs whose 128 x 128 tiles would leave CUs idle
extern "C" __global__ __launch_bounds__(256) void rtq_mm64_q4_0(FwdArgs a) { mm_tile<FMT_Q4_0, 4, RTQ_MM64_RING>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_mm64_q8_0(FwdArgs a) { mm_tile<FMT_Q8_0, 4, RTQ_MM64_RING>(a); }
// 128 rows x 32 tokens: two or more workgroups per CU where 128 x 64 tiles give about one
extern "C" __global__ __launch_bounds__(256) void rtq_mm32_q4_0(FwdArgs a) { mm_tile<FMT_Q4_0, 2, RTQ_MM32_RING>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_mm32_q8_0(FwdArgs a) { mm_tile<FMT_Q8_0, 2, RTQ_MM32_RING>(a); }

// ============================================================== forward GEMM, large grids (Q4_K / Q6_K)
// rtq_mm_*'s ring kernel for the K-quants: 128 weight rows x 16 TTN tokens (TTN 4 or 2), four
// waves, wave w owning row groups 2w, 2w+1 x all token tiles, the half-chunk operands - codes
// (Q4_K in the Q4_0 layout, Q6_K in the Q8_0 layout), the sub-block scale words of the 128 rows,
// the activation codes (Q8_K values as exact f16) - copied global -> LDS by buffer loads with an
// LDS destination into a RING-stage ring.  Arithmetic as fwd_tile's K-quant path: the 6-bit scales
// folded into the f16 weight fragments (Q4_K: sc u and m; Q6_K: sh q and sl q), two f16 MFMAs per
// block accumulate the super-block's exact integer sums S1, S2 over its four half chunks, and the
// f32 epilogue runs once per super-block: Q4_K y += (d d_x) S1 - (dmin d_x) S2, Q6_K
// y += (d d_x) (16 S1 + S2).  The super-block scales (d, dmin) of the lane's rows and the tokens'
// Q8_K d are loaded from global memory at the super-block's first half chunk and used at its last.
template <int FMT, int TTN>
struct MmkStage {  // one half chunk in LDS, in 16-byte units
  static constexpr int XQ = 0;                                           // [tt TTN][j2 2][lane 64] codes
  static constexpr int WQ = TTN * 2 * 64;                                // [rg 8][lane 64] Q4_K 8 B, Q6_K 16 B
  static constexpr int WK = WQ + (FMT == FMT_Q4_K ? 8 * 64 / 2 : 8 * 64);  // [rg 8][row 16] sub-block scale words
  static constexpr int SIZE = WK + 8 * 4;
  static constexpr int NX = 2 * TTN;
  static constexpr int NWQ = FMT == FMT_Q4_K ? 16 : 8;
};

template <int FMT, int TTN, int RING>
__device__ __forceinline__ void mmk_tile(const FwdArgs& a) {
  static_assert(TTN == 4 || TTN == 2, "64- or 32-token tiles");
  using St = MmkStage<FMT, TTN>;
  extern __shared__ u4v mm_lds[];
  const int lane = threadIdx.x & 63, li = lane & 15, g = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int Kc = a.Kp / 128, nhc = a.Kp / 64;
  const int ngroups = a.Np / 16, ntt = a.Tp / 16;
  constexpr int MM_GR = 8;
  const int nrb = (ngroups + 7) / 8, ntb = ntt / TTN, ntiles = nrb * ntb;
  const int id = blockIdx.x, xcd = id & 7, per = ntiles >> 3, rem = ntiles & 7;
  const int q = xcd * per + min(xcd, rem) + (id >> 3);
  const int gfull = nrb / MM_GR, q0 = gfull * MM_GR * ntb;
  int rb, tb;
  if (q < q0) {
    const int in = q % (MM_GR * ntb);
    rb = (q / (MM_GR * ntb)) * MM_GR + in % MM_GR;
    tb = in / MM_GR;
  } else {
    const int gr = nrb - gfull * MM_GR, in = q - q0;
    rb = gfull * MM_GR + in % gr;
    tb = in / gr;
  }
  const int rg0 = rb * 8, tt0 = tb * TTN;

  const uint32_t nb_x = (uint32_t)a.Tp * a.Kp * 2;
  const uint32_t nb_w = (uint32_t)a.Np * a.Kp / (FMT == FMT_Q4_K ? 2 : 1), nb_wd = (uint32_t)a.Np * a.Kp / 16;
  const __amdgpu_buffer_rsrc_t rs_x = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(a.xq), (short)0, nb_x, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs_w = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(a.wq), (short)0, nb_w, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs_wd = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.wd), (short)0, nb_wd, 0x00020000);
  constexpr int KX = St::NX / 4, KW = St::NWQ / 4;
  static_assert(St::NX % 4 == 0 && St::NWQ % 4 == 0, "load split over four waves");
  uint32_t vx[KX], vw[KW], ve = 0;
#pragma unroll
  for (int k = 0; k < KX; k++) {
    const int i = w + 4 * k;
    const uint32_t ttg = (uint32_t)min(tt0 + (i >> 1), ntt - 1);
    vx[k] = ((ttg * Kc * 4 + (i & 1)) * 64 + lane) * 16;
  }
#pragma unroll
  for (int k = 0; k < KW; k++) {
    const int iw = w + 4 * k;
    if (FMT == FMT_Q4_K) {
      const int wi = (iw & 1) * 64 + lane;
      const uint32_t rgg = (uint32_t)min(rg0 + (iw >> 1), ngroups - 1);
      vw[k] = ((rgg * Kc * 64 + (wi >> 1)) * 4 + (wi & 1)) * 4;
    } else {
      const uint32_t rgg = (uint32_t)min(rg0 + iw, ngroups - 1);
      vw[k] = (rgg * Kc * 2 * 64 + lane) * 16;
    }
  }
  if (w < 2) {  // sub-block scale words (blocks 2h, 2h+1): word wi -> row wi % 16 of row group wi / 16
    const int wi = w * 64 + lane;
    const uint32_t rgg = (uint32_t)min(rg0 + (wi >> 4), ngroups - 1);
    ve = ((rgg * Kc * 16 + (wi & 15)) * 2) * 4;
  }
  auto issue = [&](int st, int hc) {
    u4v* S = mm_lds + st * St::SIZE;
    const uint32_t kc = hc >> 1, h = hc & 1;
#pragma unroll
    for (int k = 0; k < KX; k++)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_x, RTQ_LDSP(S + St::XQ + (w + 4 * k) * 64), 16, vx[k], hc * 2048u, 0, 0);
#pragma unroll
    for (int k = 0; k < KW; k++) {
      const int iw = w + 4 * k;
      if (FMT == FMT_Q4_K)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_w, RTQ_LDSP(S + St::WQ + (iw >> 1) * 32 + (iw & 1) * 16), 4, vw[k],
                                                 kc * 1024u + h * 8u, 0, 0);
      else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_w, RTQ_LDSP(S + St::WQ + iw * 64), 16, vw[k], hc * 1024u, 0, 0);
    }
    if (w < 2)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_wd, RTQ_LDSP(S + St::WK + w * 16), 4, ve, kc * 128u + h * 4u, 0, 0);
  };

  const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  f4 acc[TTN][2], s1[TTN][2], s2[TTN][2];
#pragma unroll
  for (int i = 0; i < TTN; i++)
#pragma unroll
    for (int r = 0; r < 2; r++) acc[i][r] = s1[i][r] = s2[i][r] = zero;
  u4v esb[2];     // (d | dmin << 16) of rows 4g .. 4g + 3 of row groups 2w, 2w + 1, this super-block
  float xsb[TTN]; // the tokens' Q8_K d of this super-block (token li of each tile)
  auto compute = [&](int st, int hc) {
    const u4v* S = mm_lds + st * St::SIZE;
    if ((hc & 3) == 0) {  // a super-block starts: its scales, consumed at its last half chunk
      const int sb = hc >> 2;
#pragma unroll
      for (int r = 0; r < 2; r++)
        esb[r] = reinterpret_cast<const u4v*>(a.wsb)[((uint32_t)min(rg0 + 2 * w + r, ngroups - 1) * (Kc >> 1) + sb) * 4 + g];
#pragma unroll
      for (int i = 0; i < TTN; i++)
        xsb[i] = a.xd[((int64_t)(2 * sb) * a.Tp + min((tt0 + i) * 16 + li, a.Tp - 1)) * 4];
    }
#pragma unroll
    for (int j2 = 0; j2 < 2; j2++) {
      half8 f1[2], f2[2];
#pragma unroll
      for (int r = 0; r < 2; r++) {
        const int rl = 2 * w + r;
        const uint32_t kw = reinterpret_cast<const uint32_t*>(S + St::WK)[rl * 16 + li];
        const uint32_t wv = j2 ? (kw >> 16) : kw;
        if (FMT == FMT_Q4_K) {
          const u2v q2 = reinterpret_cast<const u2v*>(S + St::WQ)[rl * 64 + lane];
          const _Float16 sc = (_Float16)(float)(wv & 0x3fu), m = (_Float16)(float)((wv >> 8) & 0x3fu);
          f1[r] = q4_0_frag<0>(j2 ? q2.y : q2.x) * sc;
          const half8 mm = {m, m, m, m, m, m, m, m};
          f2[r] = mm;
        } else {
          const u4v qv = S[St::WQ + rl * 64 + lane];
          const int s0 = (int)(int8_t)(wv & 0xffu), s1v = (int)(int8_t)((wv >> 8) & 0xffu);
          const _Float16 h0 = (_Float16)(float)(s0 >> 4), h1 = (_Float16)(float)(s1v >> 4);
          const _Float16 l0 = (_Float16)(float)(s0 & 15), l1 = (_Float16)(float)(s1v & 15);
          const half8 qf = j2 ? q8_frag(qv.z, qv.w) : q8_frag(qv.x, qv.y);
          const half8 sh = {h0, h0, h0, h0, h1, h1, h1, h1}, sl = {l0, l0, l0, l0, l1, l1, l1, l1};
          f1[r] = qf * sh;
          f2[r] = qf * sl;
        }
      }
#pragma unroll
      for (int i = 0; i < TTN; i++) {
        const half8 xf = __builtin_bit_cast(half8, S[St::XQ + (i * 2 + j2) * 64 + lane]);
#pragma unroll
        for (int r = 0; r < 2; r++) {
          s1[i][r] = mfma_f16(f1[r], xf, s1[i][r]);
          s2[i][r] = mfma_f16(f2[r], xf, s2[i][r]);
        }
      }
    }
    if ((hc & 3) == 3) {  // the super-block's f32 epilogue, then the sums restart
#pragma unroll
      for (int i = 0; i < TTN; i++)
#pragma unroll
        for (int r = 0; r < 2; r++) {
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const uint32_t ev = comp(esb[r], e);
            const float dd = h2f((uint16_t)(ev & 0xffffu)) * xsb[i];
            if (FMT == FMT_Q4_K) {
              const float dm = h2f((uint16_t)(ev >> 16)) * xsb[i];
              acc[i][r][e] = fmaf(dd, s1[i][r][e], fmaf(-dm, s2[i][r][e], acc[i][r][e]));
            } else {
              acc[i][r][e] = fmaf(dd, fmaf(16.0f, s1[i][r][e], s2[i][r][e]), acc[i][r][e]);
            }
          }
          s1[i][r] = zero;
          s2[i][r] = zero;
        }
    }
  };

  static_assert(RING >= 3 && (RING - 2) * (KX + KW + 1) <= 63, "ring depth within the load counter");
  constexpr int MINL = KX + KW;
#pragma unroll
  for (int s = 0; s < RING - 1; s++)
    if (s < nhc) issue(s, s);
  for (int hc0 = 0; hc0 < nhc; hc0 += RING) {
#pragma unroll
    for (int u = 0; u < RING; u++) {
      const int hc = hc0 + u;
      if (hc < nhc) {
        vm_wait_stages<MINL>(min(RING - 2, nhc - 1 - hc));
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (hc + RING - 1 < nhc) issue((u + RING - 1) % RING, hc + RING - 1);
        compute(u, hc);
      }
    }
  }

  // ---- epilogue as rtq_mm_*: bias, LoRA up-projection per row group, y
  const bool lora = a.hp != nullptr;
  float(*sh)[RTQ_LDS_RANK + 1] = reinterpret_cast<float(*)[RTQ_LDS_RANK + 1]>(mm_lds);
  float(*sbm)[RTQ_LDS_RANK + 1] = sh + 16 * TTN;
  int span0 = 0, span1 = 0;
  int win0[2] = {0, 0}, win1[2] = {0, 0};
  if (lora) {
    rb_span(a.rb, a.r, rg0 * 16, min(rg0 * 16 + 128, a.N), span0, span1);
#pragma unroll
    for (int r = 0; r < 2; r++) rb_span(a.rb, a.r, (rg0 + 2 * w + r) * 16, (rg0 + 2 * w + r) * 16 + 16, win0[r], win1[r]);
  }
  f4 lacc[TTN][2];
#pragma unroll
  for (int i = 0; i < TTN; i++)
#pragma unroll
    for (int r = 0; r < 2; r++) lacc[i][r] = zero;
  for (int c0 = span0; c0 < span1; c0 += RTQ_LDS_RANK) {
    const int c1 = min(c0 + RTQ_LDS_RANK, span1);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    for (int j0 = c0; j0 < c1; j0 += 16) {
      float hv[8], bv[8];
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const int e = threadIdx.x + 256 * k, tl = e >> 4, j = min(j0 + (e & 15), a.r - 1);
        hv[k] = tl < 16 * TTN ? sum_partials(a.hp, (int64_t)min(tt0 * 16 + tl, a.T - 1) * a.r + j, a.nhp) : 0.0f;
        bv[k] = a.lb[(int64_t)min(rg0 * 16 + tl, a.N - 1) * a.r + j];
      }
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const int e = threadIdx.x + 256 * k, jl = j0 - c0 + (e & 15);
        if ((e >> 4) < 16 * TTN) sh[e >> 4][jl] = hv[k];
        sbm[e >> 4][jl] = bv[k];
      }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 2; r++) {
      const int lo = max(win0[r], c0), hi = min(win1[r], c1);
      const int nb0 = (rg0 + 2 * w + r) * 16, rl = (2 * w + r) * 16;
      for (int j0 = lo; j0 < hi; j0 += 4) {
        const int j = j0 + g, jl = min(j, hi - 1) - c0;
        const float bv = (nb0 + li < a.N && j < hi) ? sbm[rl + li][jl] : 0.0f;
#pragma unroll
        for (int i = 0; i < TTN; i++) {
          const float hv = (tt0 * 16 + i * 16 + li < a.T && j < hi) ? sh[i * 16 + li][jl] : 0.0f;
          lacc[i][r] = mfma_f32(bv, hv, lacc[i][r]);
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < TTN; i++) {
#pragma unroll
    for (int r = 0; r < 2; r++) {
      const int t = tt0 * 16 + i * 16 + li;
      const int nb0 = (rg0 + 2 * w + r) * 16, n0 = nb0 + 4 * g;
      if (nb0 >= a.N) continue;
      if (t < a.T) {
        f4 v = acc[i][r];
#pragma unroll
        for (int e = 0; e < 4; e++) {
          float o = v[e];
          if (a.bias) o = o + a.bias[min(n0 + e, a.N - 1)];
          if (lora) o = o + a.s * lacc[i][r][e];
          v[e] = o;
        }
        float* yr = a.y + (int64_t)t * a.N;
        if ((a.N & 3) == 0 && n0 + 3 < a.N) {
          *reinterpret_cast<f4*>(yr + n0) = v;
        } else {
#pragma unroll
          for (int e = 0; e < 4; e++)
            if (n0 + e < a.N) yr[n0 + e] = v[e];
        }
      }
    }
  }
}

extern "C" __global__ __launch_bounds__(256) void rtq_mmk64_q4_k(FwdArgs a) { mmk_tile<FMT_Q4_K, 4, RTQ_MM64_RING>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_mmk64_q6_k(FwdArgs a) { mmk_tile<FMT_Q6_K, 4, RTQ_MM64_RING>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_mmk32_q4_k(FwdArgs a) { mmk_tile<FMT_Q4_K, 2, RTQ_MM32_RING>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_mmk32_q6_k(FwdArgs a) { mmk_tile<FMT_Q6_K, 2, RTQ_MM32_RING>(a); }

// ============================================================== forward GEMM on int8 MFMA (Q4_0 / Q8_0)
// rtq_mm64_*'s tiles (128 weight rows x 16 TTN tokens, TTN 4 here, four waves, the same RING-stage
// ring of half-chunk operands copied global -> LDS by buffer loads with an LDS destination), with
// the block sums on v_mfma_i32_32x32x32_i8: wave w owns weight rows 32 w .. 32 w + 31 (row groups
// 2w, 2w+1) x all tokens, in 32 x 32 tiles, one i8 MFMA per tile and block (K = 32 = one block).
// The weight codes are the device's codes as they lie in LDS (a lane's 16 codes are those of k-groups
// 2 (l / 32), 2 (l / 32) + 1 of its row: two reads; Q8_0 needs no conversion, Q4_0 nibbles become
// u - 8 bytes with three VALU operations per four codes); the activation
// codes are act_prep's int8 fragments in the same k order (xq_i8), half the bytes of the f16 ones.
// Per tile and block: isum (i32, exact) and the scale products d_w d_x from one f16 32x32x16 MFMA
// (operands in k slot 0: an outer product, exact in f32), then acc += f32(isum) * (d_w d_x) - the
// same arithmetic as rtq_mm_*, so the outputs agree with it bit for bit.  The epilogue costs two
// VALU operations (convert, FMA) per output element and block against the f16 kernel's one FMA.
// MFMA 32 x 32 output layout: lane l holds column l % 32 (token) and rows 8 (e / 4) + 4 (l / 32) +
// e % 4, e < 16 (weight rows).
typedef int32_t i4v __attribute__((ext_vector_type(4)));
typedef int32_t i16v __attribute__((ext_vector_type(16)));

template <int FMT, int TTN>
struct MmI8Stage {  // one half chunk in LDS, in 16-byte units
  static constexpr int TT32 = TTN / 2;                // token tiles of 32
  static constexpr int XQ = 0;                        // [tt32][j2 2][lane 64] int8 codes
  static constexpr int WQ = TT32 * 2 * 64;            // [rg 8][lane 64] codes: Q8_0 16 B, Q4_0 8 B
  static constexpr int WD = WQ + (FMT == FMT_Q4_0 ? 8 * 64 / 2 : 8 * 64);  // [rg 8][row 16] fp16 scale pairs
  static constexpr int XD = WD + 8 * 4;               // [t 16 TTN] fp16 activation scale pairs
  static constexpr int NXD = TTN / 4;                 // loads of activation scales (64 tokens each)
  static constexpr int SIZE = XD + 16 * NXD;
  static constexpr int NX = 2 * TT32;                 // loads of activation fragments (1 KB each)
  static constexpr int NWQ = FMT == FMT_Q4_0 ? 16 : 8;  // loads of weight codes
};

// Q4_0 codes of a word (low nibbles: 4 elements, high nibbles: the 4 elements 16 on) -> signed
// int8 codes u - 8: (u | 0x80) - 8 per byte cannot borrow across bytes, then the sign bit flipped
__device__ __forceinline__ uint32_t q4_i8(uint32_t u) { return ((u | 0x80808080u) - 0x08080808u) ^ 0x80808080u; }

template <int FMT, int TTN, int RING>
__device__ __forceinline__ void mmi8_tile(const FwdArgs& a) {
  static_assert(TTN == 8 || TTN == 4, "128- or 64-token tiles");
  using St = MmI8Stage<FMT, TTN>;
  constexpr int TT32 = St::TT32;
  extern __shared__ u4v mm_lds[];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int Kc = a.Kp / 128, nhc = a.Kp / 64;
  const int ngroups = a.Np / 16, ntt = a.Tp / 16, ntt32 = a.Tp / 32;
  // tile order as rtq_mm_*: XCD-aware, row blocks in groups of MM_GR per token-block sweep
  constexpr int MM_GR = 8;
  const int nrb = (ngroups + 7) / 8, ntb = ntt / TTN, ntiles = nrb * ntb;
  const int id = blockIdx.x, xcd = id & 7, per = ntiles >> 3, rem = ntiles & 7;
  const int q = xcd * per + min(xcd, rem) + (id >> 3);
  const int gfull = nrb / MM_GR, q0 = gfull * MM_GR * ntb;
  int rb, tb;
  if (q < q0) {
    const int in = q % (MM_GR * ntb);
    rb = (q / (MM_GR * ntb)) * MM_GR + in % MM_GR;
    tb = in / MM_GR;
  } else {
    const int gr = nrb - gfull * MM_GR, in = q - q0;
    rb = gfull * MM_GR + in % gr;
    tb = in / gr;
  }
  const int rg0 = rb * 8, tt0 = tb * TTN;

  const uint32_t nb_x = (uint32_t)a.Tp * a.Kp, nb_xd = (uint32_t)Kc * a.Tp * 8;
  const uint32_t nb_w = (uint32_t)a.Np * a.Kp / (FMT == FMT_Q4_0 ? 2 : 1), nb_wd = (uint32_t)a.Np * a.Kp / 16;
  const __amdgpu_buffer_rsrc_t rs_x = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(a.xq), (short)0, nb_x, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs_xd = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.xdh), (short)0, nb_xd, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs_w = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(a.wq), (short)0, nb_w, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs_wd = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.wdr), (short)0, nb_wd, 0x00020000);
  constexpr int KX = St::NX / 4, KW = St::NWQ / 4;
  static_assert(St::NX % 4 == 0 && St::NWQ % 4 == 0 && St::NXD <= 2, "load split over four waves");
  uint32_t vx[KX], vw[KW], ve = 0;
#pragma unroll
  for (int k = 0; k < KX; k++) {  // activation fragments: 32-token tile i / 2, block 2h + i % 2
    const int i = w + 4 * k;
    const uint32_t ttg = (uint32_t)min(tt0 / 2 + (i >> 1), ntt32 - 1);
    vx[k] = ((ttg * Kc * 4 + (i & 1)) * 64 + lane) * 16;
  }
#pragma unroll
  for (int k = 0; k < KW; k++) {  // weight codes (as rtq_mm_*)
    const int iw = w + 4 * k;
    if (FMT == FMT_Q4_0) {  // row group iw / 2, words 64 m .. 64 m + 63 of its 128
      const int wi = (iw & 1) * 64 + lane;
      const uint32_t rgg = (uint32_t)min(rg0 + (iw >> 1), ngroups - 1);
      vw[k] = ((rgg * Kc * 64 + (wi >> 1)) * 4 + (wi & 1)) * 4;
    } else {
      const uint32_t rgg = (uint32_t)min(rg0 + iw, ngroups - 1);
      vw[k] = (rgg * Kc * 2 * 64 + lane) * 16;
    }
  }
  if (w < 2) {  // weight scale pairs: word wi -> row wi % 16 of row group wi / 16
    const int wi = w * 64 + lane;
    const uint32_t rgg = (uint32_t)min(rg0 + (wi >> 4), ngroups - 1);
    ve = ((rgg * Kc * 16 + (wi & 15)) * 2) * 4;
  } else if (w - 2 < St::NXD) {  // fp16 activation scales of blocks 2h, 2h+1: word wi -> token wi
    const int wi = (w - 2) * 64 + lane;
    ve = (uint32_t)min(tt0 * 16 + wi, a.Tp - 1) * 8;
  }
  auto issue = [&](int st, int hc) {
    u4v* S = mm_lds + st * St::SIZE;
    const uint32_t kc = hc >> 1, h = hc & 1;
#pragma unroll
    for (int k = 0; k < KX; k++)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_x, RTQ_LDSP(S + St::XQ + (w + 4 * k) * 64), 16, vx[k], hc * 2048u, 0, 0);
#pragma unroll
    for (int k = 0; k < KW; k++) {
      const int iw = w + 4 * k;
      if (FMT == FMT_Q4_0)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_w, RTQ_LDSP(S + St::WQ + (iw >> 1) * 32 + (iw & 1) * 16), 4, vw[k],
                                                 kc * 1024u + h * 8u, 0, 0);
      else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_w, RTQ_LDSP(S + St::WQ + iw * 64), 16, vw[k], hc * 1024u, 0, 0);
    }
    if (w < 2)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_wd, RTQ_LDSP(S + St::WD + w * 16), 4, ve, kc * 128u + h * 4u, 0, 0);
    else if (w - 2 < St::NXD)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_xd, RTQ_LDSP(S + St::XD + (w - 2) * 16), 4, ve,
                                               kc * (uint32_t)a.Tp * 8u + h * 4u, 0, 0);
  };

  const f16v zero16 = {};
  const i16v izero = {};
  f16v acc[TT32];
#pragma unroll
  for (int i = 0; i < TT32; i++) acc[i] = zero16;
  const int r32 = lane & 31, hl = lane >> 5;
  const int rgw = 2 * w + (r32 >> 4), rho = r32 & 15;  // this lane's A row: row rho of row group rgw
  // the scale MFMAs' operands: one value in k slot 0, the other slots zero for the whole loop
  u4v sop[2][1 + TT32];
#pragma unroll
  for (int j2 = 0; j2 < 2; j2++)
#pragma unroll
    for (int i = 0; i <= TT32; i++) sop[j2][i] = u4v{0u, 0u, 0u, 0u};
  auto compute = [&](int st) {
    const u4v* S = mm_lds + st * St::SIZE;
    i4v wa[2];
    if (FMT == FMT_Q4_0) {  // lanes rho + 32 hl, + 16 of the row group's 64: one word per block
      const u2v* W2 = reinterpret_cast<const u2v*>(S + St::WQ) + rgw * 64 + rho + 32 * hl;
      const u2v e0 = W2[0], e1 = W2[16];
#pragma unroll
      for (int j2 = 0; j2 < 2; j2++) {
        const uint32_t a0 = j2 ? e0.y : e0.x, a1 = j2 ? e1.y : e1.x;
        wa[j2] = __builtin_bit_cast(i4v, u4v{q4_i8(a0 & 0x0f0f0f0fu), q4_i8((a0 >> 4) & 0x0f0f0f0fu),
                                               q4_i8(a1 & 0x0f0f0f0fu), q4_i8((a1 >> 4) & 0x0f0f0f0fu)});
      }
    } else {  // block j of lane lam at bytes 16 lam + 8 j: one 8-byte read per half fragment
      const u2v* W2 = reinterpret_cast<const u2v*>(S + St::WQ) + 2 * (rgw * 64 + rho + 32 * hl);
#pragma unroll
      for (int j2 = 0; j2 < 2; j2++) {
        const u2v p0 = W2[j2], p1 = W2[32 + j2];
        wa[j2] = __builtin_bit_cast(i4v, u4v{p0.x, p0.y, p1.x, p1.y});
      }
    }
    // scale operands: d_w of this lane's row, d_x of its token, in k slot 0 (lanes 0 .. 31; the
    // upper lanes' words stay zero)
    const uint32_t* wdw = reinterpret_cast<const uint32_t*>(S + St::WD);
    const uint32_t* xdw = reinterpret_cast<const uint32_t*>(S + St::XD);
    if (hl == 0) {
      const uint32_t dwp = wdw[rgw * 16 + rho];
      sop[0][0].x = dwp & 0xffffu;
      sop[1][0].x = dwp >> 16;
#pragma unroll
      for (int i = 0; i < TT32; i++) {
        const uint32_t xsv = xdw[i * 32 + r32];
        sop[0][1 + i].x = xsv & 0xffffu;
        sop[1][1 + i].x = xsv >> 16;
      }
    }
#pragma unroll
    for (int i = 0; i < TT32; i++) {
#pragma unroll
      for (int j2 = 0; j2 < 2; j2++) {
        const i4v xf = __builtin_bit_cast(i4v, S[St::XQ + (i * 2 + j2) * 64 + lane]);
        const i16v c = __builtin_amdgcn_mfma_i32_32x32x32_i8(wa[j2], xf, izero, 0, 0, 0);
        const f16v sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, sop[j2][0]),
                                                              __builtin_bit_cast(half8, sop[j2][1 + i]), zero16, 0, 0, 0);
#pragma unroll
        for (int e = 0; e < 16; e++) acc[i][e] = fmaf((float)c[e], sc[e], acc[i][e]);
      }
    }
  };

  static_assert(RING >= 3 && (RING - 2) * (KX + KW + 2) <= 63, "ring depth within the load counter");
  constexpr int MINL = KX + KW + (St::NXD >= 2 ? 1 : 0);
#pragma unroll
  for (int s = 0; s < RING - 1; s++)
    if (s < nhc) issue(s, s);
  for (int hc0 = 0; hc0 < nhc; hc0 += RING) {
#pragma unroll
    for (int u = 0; u < RING; u++) {
      const int hc = hc0 + u;
      if (hc < nhc) {
        vm_wait_stages<MINL>(min(RING - 2, nhc - 1 - hc));
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (hc + RING - 1 < nhc) issue((u + RING - 1) % RING, hc + RING - 1);
        compute(u);
      }
    }
  }

  // ---- epilogue: bias, LoRA up-projection (f32 MFMA 32x32x2 in the same output layout), y.  The
  // wave's 32 rows read the ranks of their row groups' members (B is zero outside them).
  const bool lora = a.hp != nullptr;
  float(*sh)[RTQ_LDS_RANK + 1] = reinterpret_cast<float(*)[RTQ_LDS_RANK + 1]>(mm_lds);
  float(*sb)[RTQ_LDS_RANK + 1] = sh + 16 * TTN;
  int span0 = 0, span1 = 0, win0 = 0, win1 = 0;
  if (lora) {
    rb_span(a.rb, a.r, rg0 * 16, min(rg0 * 16 + 128, a.N), span0, span1);
    rb_span(a.rb, a.r, (rg0 + 2 * w) * 16, (rg0 + 2 * w) * 16 + 32, win0, win1);
  }
  f16v lacc[TT32];
#pragma unroll
  for (int i = 0; i < TT32; i++) lacc[i] = zero16;
  for (int c0 = span0; c0 < span1; c0 += RTQ_LDS_RANK) {
    const int c1 = min(c0 + RTQ_LDS_RANK, span1);
    __builtin_amdgcn_s_barrier();  // every wave is past its last read of the ring / previous chunk
    asm volatile("" ::: "memory");
    for (int j0 = c0; j0 < c1; j0 += 16) {
      float hv[8], bv[8];
#pragma unroll
      for (int k = 0; k < 8; k++) {  // rows e / 16: 16 TTN token rows of h, 128 weight rows of B
        const int e = threadIdx.x + 256 * k, tl = e >> 4, j = min(j0 + (e & 15), a.r - 1);
        hv[k] = tl < 16 * TTN ? sum_partials(a.hp, (int64_t)min(tt0 * 16 + tl, a.T - 1) * a.r + j, a.nhp) : 0.0f;
        bv[k] = a.lb[(int64_t)min(rg0 * 16 + tl, a.N - 1) * a.r + j];
      }
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const int e = threadIdx.x + 256 * k, jl = j0 - c0 + (e & 15);
        if ((e >> 4) < 16 * TTN) sh[e >> 4][jl] = hv[k];
        sb[e >> 4][jl] = bv[k];
      }
    }
    __syncthreads();
    const int lo = max(win0, c0), hi = min(win1, c1);
    const int nrow = (rg0 + 2 * w) * 16 + r32;
    for (int j0 = lo; j0 < hi; j0 += 2) {
      const int j = j0 + hl, jl = min(j, hi - 1) - c0;
      const float bv = (nrow < a.N && j < hi) ? sb[32 * w + r32][jl] : 0.0f;
#pragma unroll
      for (int i = 0; i < TT32; i++) {
        const float hv = (tt0 * 16 + i * 32 + r32 < a.T && j < hi) ? sh[i * 32 + r32][jl] : 0.0f;
        lacc[i] = __builtin_amdgcn_mfma_f32_32x32x2f32(bv, hv, lacc[i], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < TT32; i++) {
    const int t = tt0 * 16 + i * 32 + r32;
    if (t >= a.T) continue;
    float* yr = a.y + (int64_t)t * a.N;
#pragma unroll
    for (int e4 = 0; e4 < 4; e4++) {
      const int n0 = (rg0 + 2 * w) * 16 + 8 * e4 + 4 * hl;
      if (n0 >= a.N) continue;
      f4 v;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        float o = acc[i][4 * e4 + e];
        if (a.bias) o = o + a.bias[min(n0 + e, a.N - 1)];
        if (lora) o = o + a.s * lacc[i][4 * e4 + e];
        v[e] = o;
      }
      if ((a.N & 3) == 0 && n0 + 3 < a.N) {
        *reinterpret_cast<f4*>(yr + n0) = v;
      } else {
#pragma unroll
        for (int e = 0; e < 4; e++)
          if (n0 + e < a.N) yr[n0 + e] = v[e];
      }
    }
  }
}

// 128 x 64 tiles (127 VGPRs, several waves per SIMD; the 128 x 128 form of this kernel holds 300,
// one wave per SIMD, and measured 1.5x slower)
extern "C" __global__ __launch_bounds__(256) void rtq_mmi8_64_q4_0(FwdArgs a) { mmi8_tile<FMT_Q4_0, 4, RTQ_MM64_RING>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_mmi8_64_q8_0(FwdArgs a) { mmi8_tile<FMT_Q8_0, 4, RTQ_MM64_RING>(a); }

// ============================================================== forward GEMV (T <= 16)
// MFMA orientation transposed against fwd_tile: A operand = the 16 token slots x 32 columns of the
// activation fragments, B operand = 32 columns x 16 weight rows, so output lane l holds weight row
// l % 16 for tokens 4(l/16) .. 4(l/16)+3: one weight scale per lane and block.
// Q4_0 / Q8_0 weight fragments keep the f16 code bias (1024 + u, u the unsigned code): the MFMA
// accumulator is seeded with -(1024 + offset) * (sum of the token's codes in the block), computed by
// the activation prep, so the MFMA output is still the exact integer block sum (every partial is
// an integer below 2^24) and the fragment costs no subtraction.  K-quants use fwd_tile's scaled
// fragments and super-block sums.
// Workgroup = 4 waves, each owning RG row groups over the workgroup's whole K range (the runtime
// takes this kernel when the row tiles alone give a workgroup per CU: an LM head).  The activation
// fragments and the per-token block scales and seeds of the workgroup's K range are staged in LDS
// once; the weight items (one chunk of RG row groups) stream through a D-deep register ring.
// blockIdx.y splits K across workgroups in whole chunks (whole super-blocks for K-quants),
// accumulating with atomics into a y the activation prep cleared.
__device__ __forceinline__ half8 h8_from_words(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  const u4v v = {a, b, c, d};
  return __builtin_bit_cast(half8, v);
}
// nibbles of bytes 4g..4g+3 -> 1024 + nibble (low nibbles, then high nibbles)
__device__ __forceinline__ half8 nib_frag_biased(uint32_t w) {
  const uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
  return h8_from_words(bytes01_to_h2(lo), bytes23_to_h2(lo), bytes01_to_h2(hi), bytes23_to_h2(hi));
}
// int8 codes -> 1024 + (q + 128)
__device__ __forceinline__ half8 byte_frag_biased(uint32_t lo, uint32_t hi) {
  lo ^= 0x80808080u;
  hi ^= 0x80808080u;
  return h8_from_words(bytes01_to_h2(lo), bytes23_to_h2(lo), bytes01_to_h2(hi), bytes23_to_h2(hi));
}

template <int FMT>
struct GRow {                          // one row group, one chunk; lane = (row li, k-group g)
  u4v q[byte_codes(FMT) ? 2 : 1];      // codes: nibble layout (component j = block j) or byte layout (part p)
  u2v d;                               // row li, blocks 0..3: fp16 scales / K-quant sub-block words
  uint32_t e;                          // row li: K-quant super-block (d, dmin)
};

template <int FMT, int RG>
struct GSlot {
  GRow<FMT> w[RG];
};

template <int FMT, int RG, int D>
__device__ __forceinline__ void gemv_tile(const FwdArgs& a) {
  constexpr bool KQ = is_kquant(FMT), B8 = byte_codes(FMT);
  extern __shared__ __attribute__((aligned(16))) char gsm[];
  __shared__ float sh[16][RTQ_LDS_RANK + 1];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, li = lane & 15, g = lane >> 4;
  const int Kc = a.Kp / 128, ngroups = a.Np / 16;
  // this workgroup's chunk range [kcb, kce)
  const int kcb = blockIdx.y * a.kc_per_split, kce = min(kcb + a.kc_per_split, Kc), kcnt = kce - kcb;
  u4v* sX = reinterpret_cast<u4v*>(gsm);                             // [kcnt * 4][64]
  float* sG = reinterpret_cast<float*>(gsm + (size_t)kcnt * 4 * 64 * 16);  // [kcnt * 4][2][16]
  // this wave's rows, over chunks [c0, c0 + nit)
  const int rg0 = (blockIdx.x * 4 + w) * RG;
  const int c0 = kcb, nit = kcnt;
  int rgc[RG];
#pragma unroll
  for (int r = 0; r < RG; r++) rgc[r] = min(rg0 + r, ngroups - 1);
  const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  f4 acc[RG], s1[KQ ? RG : 1], s2[KQ ? RG : 1];
#pragma unroll
  for (int r = 0; r < RG; r++) acc[r] = zero;
  if (KQ) {
#pragma unroll
    for (int r = 0; r < (KQ ? RG : 1); r++) s1[r] = s2[r] = zero;
  }
  const bool lead = blockIdx.y == 0;
  const bool lora = a.hp && lead;

  auto issue = [&](GSlot<FMT, RG>& S, int it) {
    const int kc = min(c0 + min(it, max(nit - 1, 0)), Kc - 1);  // clamped: always a valid chunk
#pragma unroll
    for (int r = 0; r < RG; r++) {
      const uint32_t base = (uint32_t)rgc[r] * Kc + kc;
      if (B8) {
        S.w[r].q[0] = reinterpret_cast<const u4v*>(a.wq)[(base * 2) * 64 + lane];
        S.w[r].q[B8 ? 1 : 0] = reinterpret_cast<const u4v*>(a.wq)[(base * 2 + 1) * 64 + lane];
      } else {
        S.w[r].q[0] = reinterpret_cast<const u4v*>(a.wq)[base * 64 + lane];
      }
      S.w[r].d = reinterpret_cast<const u2v*>(a.wdr)[base * 16 + li];
      if (KQ) S.w[r].e = a.wsb[((uint32_t)rgc[r] * (Kc >> 1) + (kc >> 1)) * 16 + li];
    }
  };
  GSlot<FMT, RG> sl[D];
#pragma unroll
  for (int s = 0; s < D - 1; s++) issue(sl[s], s);

  // stage the activation fragments and token scales / seeds of chunks [kcb, kce)
  {
    const u4v* XQ = reinterpret_cast<const u4v*>(a.xq);
    const int nx = kcnt * 4 * 64;
    for (int i = threadIdx.x; i < nx; i += 256) sX[i] = XQ[(size_t)kcb * 4 * 64 + i];
    const u4v* XG = reinterpret_cast<const u4v*>(a.xg);
    const int ng = kcnt * 4 * 2 * 4;
    for (int i = threadIdx.x; i < ng; i += 256) reinterpret_cast<u4v*>(sG)[i] = XG[(size_t)kcb * 4 * 2 * 4 + i];
    if (lora)  // the runtime takes this kernel for ranks up to RTQ_LDS_RANK only
      for (int e = threadIdx.x; e < 16 * a.r; e += 256) {
        const int t = e / a.r, j = e % a.r;
        sh[t][j] = t < a.T ? sum_partials(a.hp, (int64_t)t * a.r + j, a.nhp) : 0.0f;
      }
  }
  __syncthreads();

  auto compute = [&](const GSlot<FMT, RG>& S, int it) {
    const int kc = c0 + it, kl = kc - kcb;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const half8 xf = __builtin_bit_cast(half8, sX[(kl * 4 + j) * 64 + lane]);
      if constexpr (!KQ) {
        const f4 dxv = *reinterpret_cast<const f4*>(&sG[((kl * 4 + j) * 2) * 16 + 4 * g]);
        const f4 seed = *reinterpret_cast<const f4*>(&sG[((kl * 4 + j) * 2 + 1) * 16 + 4 * g]);
#pragma unroll
        for (int r = 0; r < RG; r++) {
          half8 wf;
          if (B8) {
            const u4v& qq = S.w[r].q[j >> 1];
            wf = (j & 1) ? byte_frag_biased(qq.z, qq.w) : byte_frag_biased(qq.x, qq.y);
          } else {
            wf = nib_frag_biased(comp(S.w[r].q[0], j));
          }
          const f4 c = mfma_f16(xf, wf, seed);
          const float dw = h2f(hcomp(S.w[r].d, j));
#pragma unroll
          for (int e = 0; e < 4; e++) acc[r][e] = fmaf(c[e], dw * dxv[e], acc[r][e]);
        }
      } else {
#pragma unroll
        for (int r = 0; r < RG; r++) {
          const uint32_t wv = hcomp(S.w[r].d, j);
          half8 f1, f2;
          if (FMT == FMT_Q4_K) {
            const _Float16 sc = (_Float16)(float)(wv & 0x3fu), m = (_Float16)(float)((wv >> 8) & 0x3fu);
            f1 = q4_0_frag<0>(comp(S.w[r].q[0], j)) * sc;
            const half8 mm = {m, m, m, m, m, m, m, m};
            f2 = mm;
          } else {
            const int sa = (int)(int8_t)(wv & 0xffu), sb = (int)(int8_t)((wv >> 8) & 0xffu);
            const _Float16 h0 = (_Float16)(float)(sa >> 4), h1 = (_Float16)(float)(sb >> 4);
            const _Float16 l0 = (_Float16)(float)(sa & 15), l1 = (_Float16)(float)(sb & 15);
            const u4v& qq = S.w[r].q[j >> 1];
            const half8 qf = (j & 1) ? q8_frag(qq.z, qq.w) : q8_frag(qq.x, qq.y);
            const half8 sh8 = {h0, h0, h0, h0, h1, h1, h1, h1}, sl8 = {l0, l0, l0, l0, l1, l1, l1, l1};
            f1 = qf * sh8;
            f2 = qf * sl8;
          }
          s1[r] = mfma_f16(xf, f1, s1[r]);
          s2[r] = mfma_f16(xf, f2, s2[r]);
        }
      }
    }
    if constexpr (KQ) {
      if (kc & 1) {  // last chunk of the super-block
        const f4 dxv = *reinterpret_cast<const f4*>(&sG[((kl * 4) * 2) * 16 + 4 * g]);  // the super-block's d_x
#pragma unroll
        for (int r = 0; r < RG; r++) {
          const uint32_t ev = S.w[r].e;
          const float dsb = h2f((uint16_t)(ev & 0xffffu));
#pragma unroll
          for (int e = 0; e < 4; e++) {
            if (FMT == FMT_Q4_K) {
              const float dm = h2f((uint16_t)(ev >> 16)) * dxv[e];
              acc[r][e] = fmaf(dsb * dxv[e], s1[r][e], fmaf(-dm, s2[r][e], acc[r][e]));
            } else {
              acc[r][e] = fmaf(dsb * dxv[e], fmaf(16.0f, s1[r][e], s2[r][e]), acc[r][e]);
            }
          }
          s1[r] = zero;
          s2[r] = zero;
        }
      }
    }
  };
  for (int it0 = 0; it0 < nit; it0 += D) {
#pragma unroll
    for (int s = 0; s < D; s++) {
      issue(sl[(s + D - 1) % D], it0 + s + D - 1);
      __builtin_amdgcn_sched_barrier(0);
      if (it0 + s < nit) compute(sl[s], it0 + s);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  const bool split = gridDim.y > 1;
#pragma unroll
  for (int r = 0; r < RG; r++) {
    const int n = (rg0 + r) * 16 + li;
    if (rg0 + r >= ngroups || n >= a.N) continue;
    float lo[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (lora) {  // LoRA up: sum_j B[n][j] h[t][j] (src/linear.rs:86); rank <= RTQ_LDS_RANK here
      for (int j0 = 0; j0 < a.r; j0 += 16) {
        float bv[16];  // sixteen independent loads of B's row n in flight
#pragma unroll
        for (int q = 0; q < 16; q++) bv[q] = a.lb[(int64_t)n * a.r + min(j0 + q, a.r - 1)];
#pragma unroll
        for (int q = 0; q < 16; q++)
          if (j0 + q < a.r)
#pragma unroll
            for (int e = 0; e < 4; e++) lo[e] = fmaf(bv[q], sh[4 * g + e][j0 + q], lo[e]);
      }
    }
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int t = 4 * g + e;
      if (t >= a.T) continue;
      float o = acc[r][e];
      if (a.bias && lead) o = o + a.bias[n];
      if (lora) o = o + a.s * lo[e];
      float* yp = a.y + (int64_t)t * a.N + n;
      if (split)
        atomicAdd(yp, o);
      else
        *yp = o;
    }
  }
}

// Q4 layouts: 4 row groups per wave; byte layouts: 2; 4-deep ring.
#define RTQ_GEMV(NAME, FMT, RG, D)                                         \
  extern "C" __global__ __launch_bounds__(256) void NAME(FwdArgs a) {      \
    gemv_tile<FMT, RG, D>(a);                                              \
  }
RTQ_GEMV(rtq_gemv_q4_0, FMT_Q4_0, 4, 4)
RTQ_GEMV(rtq_gemv_q8_0, FMT_Q8_0, 2, 4)
// (Q4_K, Q6_K: 2-deep rings, Q6_K held to five waves per SIMD (96 VGPRs), so that an LM head's 594 /
// 1187 workgroups are resident in one round; at 16 tokens Q4_K 42.6 -> 39.5 us, Q6_K 51.3 -> 49.0;
// Q8_0 measured slower so: 43.1 -> 44.2)
RTQ_GEMV(rtq_gemv_q4_k, FMT_Q4_K, 4, 2)
extern "C" __global__ __launch_bounds__(256, 5) void rtq_gemv_q6_k(FwdArgs a) { gemv_tile<FMT_Q6_K, 2, 2>(a); }

// ============================================================== forward GEMV for T <= 4, one launch
// y = x W^T (+ bias) (+ s (x A^T) B^T) for T <= NT tokens (NT 1 or 4).  Each workgroup first
// quantises x into LDS with the activation kernel's arithmetic (Q8_0 per 32 columns for Q4_0 /
// Q8_0 weights, Q8_K per 256 for the K-quants: the same codes and scales bit for bit), forms
// h = x A^T there when adapted, then each wave streams its row tiles (RG row groups of 16 rows over
// every chunk; tiles v, v + waves, .. for wave v) through a D-deep register ring that runs on
// across tiles.  Lane (row li, k-group g) holds, per block j of a chunk, the codes of elements
// 32j + 4g .. + 3 and 32j + 16 + 4g .. + 3 (the device layout): two v_dot4_i32_i8 with the
// activation codes of the same elements (laid out in LDS per (token, chunk, k-group): 32 bytes)
// give its share of the block's integer sum, exactly.  Q4_0 / Q8_0: each lane accumulates its
// shares times the block's d_w d_x in f32 (Q4_0's code offset -8 enters as 8 times the lane's
// activation code sum, kept in LDS per block), and the four k-groups' sums are added across
// lanes once per tile (a fixed order; within 1e-6 of rtq_gemv_*, which adds the block's whole
// integer sum first).  K-quants: the super-block sums S1, S2 are exact integers added across lanes
// once per super-block, then rtq_gemv_*'s epilogue operation for operation (the same bits).  The
// four lanes of a row hold the same sums; lane g stores token g.
template <int FMT, int RG, int D, int NT>
__device__ __forceinline__ void gemvq(const GemvqArgs& a) {
  constexpr bool KQ = is_kquant(FMT), B8 = byte_codes(FMT);
  extern __shared__ __attribute__((aligned(16))) char gqs[];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, li = lane & 15, g = lane >> 4;
  const int nw = (int)(blockDim.x >> 6), Kc = a.Kp / 128, Kb = a.Kp / 32, ngroups = a.Np / 16;
  uint32_t* xs = reinterpret_cast<uint32_t*>(gqs);                       // [NT][Kc][4 g][4 j][2]
  float* sdx = reinterpret_cast<float*>(gqs + (size_t)NT * a.Kp);        // [NT][Kb] block scales
  int* ssum = reinterpret_cast<int*>(sdx + NT * Kb);                     // [NT][Kb]: code sums (Q4_0: 8 x
                                                                         //   the k-group's, [NT][Kc][4 g][4 j])
  float* sh = reinterpret_cast<float*>(ssum + NT * Kb * (FMT == FMT_Q4_0 ? 4 : 1));  // [NT][RTQ_LDS_RANK] h
  // ---- the weight stream: its first D - 1 items are requested before the activation work
  // (the wave index through readfirstlane: the tile and chunk arithmetic stays scalar)
  const int wv = blockIdx.x * nw + __builtin_amdgcn_readfirstlane(w), nwv = gridDim.x * nw;
  const int ntw = wv < a.ntiles ? min(a.tiles_per_wave, (a.ntiles - wv + nwv - 1) / nwv) : 0;
  const int nit = ntw * Kc;
  auto item = [&](int it, int& tile, int& kc) {
    const int c = min(it, max(nit - 1, 0));  // clamped: always a real item
    tile = wv + (c / Kc) * nwv;
    kc = c % Kc;
  };
  // buffer loads: a per-lane offset and a per-item scalar one (the weight is below 4 GB: the caller checks)
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.wq, (uint32_t)ngroups * Kc * 1024u * (B8 ? 2u : 1u));
  const __amdgpu_buffer_rsrc_t rd = make_rsrc(a.wdr, (uint32_t)ngroups * Kc * 128u);
  const __amdgpu_buffer_rsrc_t re = make_rsrc(a.wsb, KQ ? (uint32_t)ngroups * (Kc >> 1) * 64u : 0u);
  auto issue = [&](GSlot<FMT, RG>& S, int it) {
    int tile, kc;
    item(it, tile, kc);
#pragma unroll
    for (int r = 0; r < RG; r++) {
      const uint32_t rg = (uint32_t)min(tile * RG + r, ngroups - 1), base = rg * Kc + kc;
      if (B8) {
        S.w[r].q[0] = __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(rq, lane * 16u, base * 2048u, 0));
        S.w[r].q[B8 ? 1 : 0] = __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(rq, lane * 16u, base * 2048u + 1024u, 0));
      } else {
        S.w[r].q[0] = __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(rq, lane * 16u, base * 1024u, 0));
      }
      S.w[r].d = __builtin_bit_cast(u2v, __builtin_amdgcn_raw_buffer_load_b64(rd, li * 8u, base * 128u, 0));
      if (KQ) S.w[r].e = __builtin_amdgcn_raw_buffer_load_b32(re, li * 4u, (rg * (Kc >> 1) + (kc >> 1)) * 64u, 0);
    }
  };
  GSlot<FMT, RG> sl[D];
  // (Q4_K at T = 1: one item fewer in flight during the activation work, the last issued after it,
  // so that the kernel fits five waves per SIMD)
  constexpr int PRE = (FMT == FMT_Q4_K && NT == 1) ? D - 2 : D - 1;
#pragma unroll
  for (int s0 = 0; s0 < PRE; s0++) issue(sl[s0], s0);
  // ---- activation codes: one 32-column block (token t, block b) per thread and pass
  for (int u0 = 0; u0 < NT * Kb; u0 += (int)blockDim.x) {
    const int u = u0 + tid, t = u / Kb, b = u % Kb, k0 = 32 * b;
    const bool real = u < NT * Kb && t < a.T && k0 < a.K;  // K % 32 == 0: a block is in or out
    float v[32];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      f4 q = {0.0f, 0.0f, 0.0f, 0.0f};
      if (real) q = reinterpret_cast<const f4*>(a.x + (int64_t)t * a.K + k0)[i];
      v[4 * i] = q.x;
      v[4 * i + 1] = q.y;
      v[4 * i + 2] = q.z;
      v[4 * i + 3] = q.w;
    }
    int q[32];
    float dstore;
    if (!KQ) {  // Q8_0: d = amax / 127, codes round(x / d) (half away from zero)
      float amax = 0.0f;
#pragma unroll
      for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
      const float d = __fdiv_rn(amax, 127.0f);
      const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
#pragma unroll
      for (int i = 0; i < 32; i++) q[i] = (int)roundf(__fmul_rn(v[i], id));
      dstore = (float)(_Float16)d;
    } else {
      // Q8_K: the first element of largest |x| of the super-block (eight adjacent lanes: larger
      // |x| wins, equal |x| the lower column), iscale = -127 / that element, codes
      // min(127, rint(iscale x)) (half to even), d = 1 / iscale
      float best = 0.0f, bmax = 0.0f;
      int bi = 0;
#pragma unroll
      for (int i = 0; i < 32; i++) {
        const float ax = fabsf(v[i]);
        if (ax > best) {
          best = ax;
          bmax = v[i];
          bi = i;
        }
      }
      bi += k0;
#pragma unroll
      for (int m = 1; m < 8; m <<= 1) {
        const float ob = __shfl_xor(best, m), om = __shfl_xor(bmax, m);
        const int oi = __shfl_xor(bi, m);
        if (ob > best || (ob == best && oi < bi)) {
          best = ob;
          bmax = om;
          bi = oi;
        }
      }
      const float iscale = best != 0.0f ? __fdiv_rn(-127.0f, bmax) : 0.0f;
#pragma unroll
      for (int i = 0; i < 32; i++) q[i] = (int)fminf(127.0f, rintf(__fmul_rn(iscale, v[i])));
      dstore = best != 0.0f ? __fdiv_rn(1.0f, iscale) : 0.0f;
    }
    if (u < NT * Kb) {
      int cs = 0;
#pragma unroll
      for (int i = 0; i < 32; i++) cs += q[i];
      const int kc = b >> 2, j = b & 3;
#pragma unroll
      for (int gg = 0; gg < 4; gg++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const int e = 16 * h + 4 * gg;
          xs[(((t * Kc + kc) * 4 + gg) * 4 + j) * 2 + h] =
              ((uint32_t)q[e] & 0xffu) | (((uint32_t)q[e + 1] & 0xffu) << 8) | (((uint32_t)q[e + 2] & 0xffu) << 16) |
              ((uint32_t)q[e + 3] << 24);
        }
      sdx[t * Kb + b] = real ? dstore : 0.0f;
      if (FMT == FMT_Q4_0) {  // 8 x (codes of k-group gg in this block), at [t][kc][gg][j]
#pragma unroll
        for (int gg = 0; gg < 4; gg++) {
          int sg = 0;
#pragma unroll
          for (int h = 0; h < 2; h++)
#pragma unroll
            for (int i = 0; i < 4; i++) sg += q[16 * h + 4 * gg + i];
          ssum[((t * Kc + kc) * 4 + gg) * 4 + j] = real ? 8 * sg : 0;
        }
      } else {
        ssum[t * Kb + b] = real ? cs : 0;
      }
    }
  }
  // ---- h = x A^T (LoRA down, f32): wave w takes pairs (t, j) w, w + nw, ..; lanes stride over K
  if (a.la) {
    for (int pr = w; pr < a.T * a.r; pr += nw) {
      const int t = pr / a.r, j = pr % a.r;
      const float* xr = a.x + (int64_t)t * a.K;
      const float* ar = a.la + (int64_t)j * a.K;
      float acc = 0.0f;
      for (int k = lane; k < a.K; k += 64) acc = fmaf(xr[k], ar[k], acc);
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) acc += __shfl_xor(acc, m);
      if (lane == 0) sh[t * RTQ_LDS_RANK + j] = acc;
    }
  }
  __syncthreads();
#pragma unroll
  for (int s0 = PRE; s0 < D - 1; s0++) issue(sl[s0], s0);

  float acc[RG][NT];
  int s1[KQ ? RG : 1][NT], s2[KQ ? RG : 1][NT];
#pragma unroll
  for (int r = 0; r < RG; r++)
#pragma unroll
    for (int t = 0; t < NT; t++) acc[r][t] = 0.0f;
#pragma unroll
  for (int r = 0; r < (KQ ? RG : 1); r++)
#pragma unroll
    for (int t = 0; t < NT; t++) s1[r][t] = s2[r][t] = 0;
  auto compute = [&](const GSlot<FMT, RG>& S, int it) {
    int tile, kc;
    item(it, tile, kc);
    u4v xv[NT][2];  // this k-group's codes of the chunk: block j at words 2j (low four), 2j + 1
    f4 xd[NT];      // the chunk's block scales
    u4v x8[NT];     // Q4_0: 8 x this k-group's code sums of the chunk's blocks
#pragma unroll
    for (int t = 0; t < NT; t++) {
      const u4v* xp = reinterpret_cast<const u4v*>(xs + ((t * Kc + kc) * 4 + g) * 8);
      xv[t][0] = xp[0];
      xv[t][1] = xp[1];
      xd[t] = *reinterpret_cast<const f4*>(sdx + t * Kb + kc * 4);
      if (FMT == FMT_Q4_0) x8[t] = *reinterpret_cast<const u4v*>(ssum + ((t * Kc + kc) * 4 + g) * 4);
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int b = kc * 4 + j;
#pragma unroll
      for (int r = 0; r < RG; r++) {
        uint32_t lo, hi;
        if (B8) {
          const u4v& qq = S.w[r].q[j >> 1];
          lo = (j & 1) ? qq.z : qq.x;
          hi = (j & 1) ? qq.w : qq.y;
        } else {
          const uint32_t cw = comp(S.w[r].q[0], j);
          lo = cw & 0x0f0f0f0fu;
          hi = (cw >> 4) & 0x0f0f0f0fu;
        }
        const uint32_t wvd = hcomp(S.w[r].d, j);
#pragma unroll
        for (int t = 0; t < NT; t++) {
          const uint32_t xl = comp(xv[t][j >> 1], 2 * (j & 1)), xh = comp(xv[t][j >> 1], 2 * (j & 1) + 1);
          if constexpr (!KQ) {  // this k-group's share of the block sum (Q4_0: codes u - 8)
            const int x0 = FMT == FMT_Q4_0 ? -(int)comp(x8[t], j) : 0;
            const int is = __builtin_amdgcn_sdot4((int)hi, (int)xh, __builtin_amdgcn_sdot4((int)lo, (int)xl, x0, false), false);
            acc[r][t] = fmaf((float)is, h2f((uint16_t)wvd) * xd[t][j], acc[r][t]);
          } else {
          if constexpr (FMT == FMT_Q4_K) {  // sc * sum u x (24-bit products); m * sum x of block g below
            const int d2 = __builtin_amdgcn_sdot4((int)hi, (int)xh, __builtin_amdgcn_sdot4((int)lo, (int)xl, 0, false), false);
            s1[r][t] += __mul24((int)(wvd & 0x3fu), d2);
          } else {
            const int dl = __builtin_amdgcn_sdot4((int)lo, (int)xl, 0, false);
            const int dh = __builtin_amdgcn_sdot4((int)hi, (int)xh, 0, false);
            const int sa = (int)(int8_t)(wvd & 0xffu), sb = (int)(int8_t)((wvd >> 8) & 0xffu);
            s1[r][t] += __mul24(sa >> 4, dl) + __mul24(sb >> 4, dh);  // sc = 16 (sc >> 4) + (sc & 15)
            s2[r][t] += __mul24(sa & 15, dl) + __mul24(sb & 15, dh);
          }
          }
        }
      }
    }
    if constexpr (FMT == FMT_Q4_K) {  // m_j * (sum of block j's codes) for block j = g, once per block
#pragma unroll
      for (int r = 0; r < RG; r++) {
        const uint32_t dw2 = (g & 2) ? S.w[r].d.y : S.w[r].d.x, wvg = (g & 1) ? dw2 >> 16 : dw2;
#pragma unroll
        for (int t = 0; t < NT; t++) s2[r][t] += __mul24((int)((wvg >> 8) & 0x3fu), ssum[t * Kb + kc * 4 + g]);
      }
    }
    if constexpr (KQ) {
      if (kc & 1) {  // last chunk of the super-block
#pragma unroll
        for (int r = 0; r < RG; r++) {
          const uint32_t ev = S.w[r].e;
          const float dsb = h2f((uint16_t)(ev & 0xffffu));
#pragma unroll
          for (int t = 0; t < NT; t++) {
            int v1 = s1[r][t], v2 = s2[r][t];
            v1 += __shfl_xor(v1, 16);
            v1 += __shfl_xor(v1, 32);
            v2 += __shfl_xor(v2, 16);
            v2 += __shfl_xor(v2, 32);
            const float dxv = sdx[t * Kb + kc * 4];
            if (FMT == FMT_Q4_K) {
              const float dm = h2f((uint16_t)(ev >> 16)) * dxv;
              acc[r][t] = fmaf(dsb * dxv, (float)v1, fmaf(-dm, (float)v2, acc[r][t]));
            } else {
              acc[r][t] = fmaf(dsb * dxv, fmaf(16.0f, (float)v1, (float)v2), acc[r][t]);
            }
            s1[r][t] = s2[r][t] = 0;
          }
        }
      }
    }
    if (kc == Kc - 1) {  // the tile's last chunk: y (+ bias) (+ LoRA up), lane g storing token g
#pragma unroll
      for (int r = 0; r < RG; r++) {
        const int n = (tile * RG + r) * 16 + li;
#pragma unroll
        for (int t = 0; t < NT; t++) {
          if constexpr (!KQ) {  // the four k-groups' sums: (g0 + g1) + (g2 + g3)
            acc[r][t] += __shfl_xor(acc[r][t], 16);
            acc[r][t] += __shfl_xor(acc[r][t], 32);
          }
          if (g == t && t < a.T && n < a.N && it < nit) {
            float o = acc[r][t];
            if (a.bias) o = o + a.bias[n];
            if (a.la) {
              float lo = 0.0f;
              for (int j = 0; j < a.r; j++)
                if (rb_keep(a.rb, n, j)) lo = fmaf(a.lb[(int64_t)n * a.r + j], sh[t * RTQ_LDS_RANK + j], lo);
              o = o + a.s * lo;
            }
            a.y[(int64_t)t * a.N + n] = o;
          }
          acc[r][t] = 0.0f;
        }
      }
    }
  };
  for (int it0 = 0; it0 < nit; it0 += D) {
#pragma unroll
    for (int s0 = 0; s0 < D; s0++) {
      issue(sl[(s0 + D - 1) % D], it0 + s0 + D - 1);
      __builtin_amdgcn_sched_barrier(0);
      if (it0 + s0 < nit) compute(sl[s0], it0 + s0);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// nibble layouts: RTQ_GQ_RG4 row groups per tile; byte layouts: RTQ_GQ_RG8; NT = 1 or 4 tokens
#define RTQ_GEMVQ(NAME, FMT, RG, NT)                                       \
  extern "C" __global__ __launch_bounds__(256) void NAME(GemvqArgs a) {    \
    gemvq<FMT, RG, RTQ_GQ_D, NT>(a);                                       \
  }
RTQ_GEMVQ(rtq_gemvq1_q4_0, FMT_Q4_0, RTQ_GQ_RG4, 1)
RTQ_GEMVQ(rtq_gemvq1_q8_0, FMT_Q8_0, RTQ_GQ_RG8, 1)
RTQ_GEMVQ(rtq_gemvq1_q4_k, FMT_Q4_K, RTQ_GQ_RG4, 1)
RTQ_GEMVQ(rtq_gemvq1_q6_k, FMT_Q6_K, RTQ_GQ_RG8, 1)
RTQ_GEMVQ(rtq_gemvq4_q4_0, FMT_Q4_0, RTQ_GQ_RG4, 4)
RTQ_GEMVQ(rtq_gemvq4_q8_0, FMT_Q8_0, RTQ_GQ_RG8, 4)
RTQ_GEMVQ(rtq_gemvq4_q4_k, FMT_Q4_K, RTQ_GQ_RG4, 4)
RTQ_GEMVQ(rtq_gemvq4_q6_k, FMT_Q6_K, RTQ_GQ_RG8, 4)
#undef RTQ_GEMVQ

// ============================================================== backward preparation
// LoRA partial products of src/linear.rs:106-111, 256 threads per workgroup, grid
// (ceil(T / 16), nhq + ngq) offset by y0 (nhq 0: the forward kept the h partials):
//   grid row y < nhq:     h partial over columns [256y, 256y + 256) of x . A^T for the 16 tokens
//                         16x .. 16x + 15 -> hp[(t * r + j) * nhq + y] (slice index fastest);
//   grid row y = nhq + q: g partial over rows [256q, 256q + 256) of dy . B for the gtok (64, 32 or 16)
//                         tokens gtok x .. -> gp[(q * T + t) * r + j] (slice-major); workgroups
//                         with gtok x >= T exit.
// The dx kernel's extra workgroups sum the partials in slice order (h, and g scaled by s).
extern "C" __global__ __launch_bounds__(256) void rtq_bwd_prep(BwdPrepArgs a) {
  constexpr int KQ = RTQ_ACT_KQ, LDX = KQ + 1;
  constexpr int SM = 16 * KQ + 64 > 16 * LDX ? 16 * KQ + 64 : 16 * LDX;  // A tile, or B slice (padded rows)
  __shared__ float sx[16 * LDX];
  __shared__ float sm[SM];
  __shared__ float red[4 * 256];
  const int y = (int)blockIdx.y + a.y0;
  if (y < a.nhq) {
    lora_partial(a.x, a.T, a.K, a.A, a.K, a.r, y * KQ, a.K, blockIdx.x * 16, a.hp, a.nhq, y, sx, sm, red);
  } else {
    const int t0 = blockIdx.x * a.gtok;
    if (t0 >= a.T) return;  // whole workgroup
    if (a.gtok == 64)
      lora_up_partial<64>(a, t0, y - a.nhq, sm, red);
    else if (a.gtok == 32)
      lora_up_partial<32>(a, t0, y - a.nhq, sm, red);
    else
      lora_up_partial<16>(a, t0, y - a.nhq, sm, red);
  }
}

// ============================================================== dx = dy . W
// Workgroup: 8 waves, tile 64 tokens x 128 columns (one K chunk); wave (wt, wk) owns 32 tokens x
// 32 columns (2 x 2 MFMA tiles).  Rows of W are split over workgroups; each split writes its own
// partial tile (plain stores; rtq_bwd_finish sums the splits in order).  Per 32-row step the
// workgroup stages, double buffered in LDS, f16 hi / lo MFMA operands:
//   * dy[64 x 32]: each thread loads one float4, scales it by 2^e (e per token row and split, so
//     that the split's largest |dy| of the row lands in [2^14, 2^15): the f16 range holds every
//     value of the row) and splits it into hi = f16 (round toward zero) and lo = f16 of the rest;
//   * W[32 x 128]: Q4_0 / Q8_0 d * q exactly as hi = f16(d * q) and lo = d * q - hi (packed f16
//     multiply and fused multiply-add on the two rows a thread converts: the residual of an f16
//     product is exact); K-quants: the f32 value of ggml's dequantisation ((d*sc)*u - dmin*m, or
//     (d*sc)*q) split like dy.  Stored transposed ([k][n]), so a lane reads its B fragment (8
//     consecutive rows of one column) in 16 bytes.
// Three f16 MFMAs per product (dh.wh + dl.wh + dh.wl): the missing dl.wl term and the rounding
// of dl leave a relative error near 2^-21 per product; the partial is scaled back by 2^-e (exact).
// Weights whose values could reach 2^15 are pre-scaled by 2^-sigma (wsc) and scaled back in the
// same multiply (wunsc); sigma is 0 for every realistic weight.
// Global loads go through buffer descriptors: a per-thread 32-bit offset plus a per-step scalar
// offset, with out-of-range reads (tokens >= T) returning zero.  A register ring keeps the loads
// D - 1 steps ahead of the MFMAs.
// W staging: thread -> half hh = tid/256 (hh 0: elements 4gg..4gg+3 of the block, hh 1:
// 16+4gg..16+4gg+3), row group rgl, rows 2p, 2p+1, k-group gg and block jb, ordered so the code
// words a wave loads lie in one 512-byte span; the two rows' scales are adjacent (one load).
// The converted pair of rows goes to LDS as one 32-bit word per column.  Within a column the
// 8-row groups are XOR-swizzled by the block index so the four blocks' writes use different banks.

template <int FMT, int NQ = 1>
struct DxSlot {
  f4 dy[NQ];
  uint32_t q[2];  // the four codes this thread converts, of rows 2p and 2p+1
  uint32_t d;     // fp16 scales of rows 2p (low half) and 2p+1 (high half)
};
template <int NQ>
struct DxSlot<FMT_Q4_K, NQ> {
  f4 dy[NQ];
  uint32_t q[2];
  u4v k;  // sub-block scale words of rows 2p (x: blocks 0, 1; y: 2, 3) and 2p+1 (z, w)
  u2v e;  // super-block (d, dmin) of rows 2p, 2p+1
};
template <int NQ>
struct DxSlot<FMT_Q6_K, NQ> : DxSlot<FMT_Q4_K, NQ> {};

// h = sum of hp, g = s * sum of gp, both in slice order (src/linear.rs:106-111), by the nfin
// finaliser workgroups of a dx grid (rel: this workgroup's index among them)
__device__ __forceinline__ void dx_lora_sums(const DxArgs& a, int rel, int nfin) {
  const int64_t n = (int64_t)a.T * a.r;
  const int64_t nthr = (int64_t)nfin * blockDim.x;
  for (int64_t e = (int64_t)rel * blockDim.x + threadIdx.x; e < n; e += nthr) {
    a.h[e] = sum_partials(a.hp, e, a.nhq);
    a.g[e] = a.s * sum_slices(a.gp, e, a.ngq, n);
  }
}

// dequantisation of the unsigned byte codes of one row, value fmaf(u, d, m):
//   Q4_0 (nibble - 8) d;  Q8_0 ((q ^ 0x80) - 128) d;  Q4_K (d sc) u - dmin m;
//   Q6_K ((q ^ 0x80) - 128) (d sc), sc of the 16-element half hh
// d16: fp16 scale (Q4_0, Q8_0); kw: the row's sub-block scale words of blocks 2h, 2h+1 of the chunk
// (h = jb / 2), ev: its super-block (d, dmin) (K-quants)
template <int FMT>
__device__ __forceinline__ void dq_params(uint32_t d16, uint32_t kw, uint32_t ev, int jb, int hh, float& d, float& m) {
  if constexpr (is_kquant(FMT)) {
    kw >>= 16 * (jb & 1);
    const float dsb = h2f((uint16_t)(ev & 0xffffu));
    if (FMT == FMT_Q4_K) {
      d = dsb * (float)(kw & 0x3fu);  // exact products
      m = -(h2f((uint16_t)(ev >> 16)) * (float)((kw >> 8) & 0x3fu));
    } else {
      d = dsb * (float)(int)(int8_t)((kw >> (8 * hh)) & 0xffu);
      m = -128.0f * d;
    }
  } else {
    d = h2f((uint16_t)d16);
    m = (FMT == FMT_Q4_0 ? -8.0f : -128.0f) * d;
  }
}

// TW: tokens per workgroup.  64: wave (wt, wk) = (w / 4, w % 4) owns 32 tokens x 32 columns
// (2 x 2 MFMA tiles).  256 (large T): wave (wt, wk) = (w / 2, w % 2) owns 64 tokens x 64 columns
// (4 x 4 tiles), so each dequantised weight element feeds four times the MFMAs; the partials keep
// the 64-token fragment order of the TW = 64 kernel.
template <int FMT, int TW>
__device__ __forceinline__ void dx_tile(const DxArgs& a) {
  // Flat grid, XCD-aware: consecutive workgroup ids go to the 8 XCDs in turn, so id % 8 selects
  // a group of row splits and all (token tile, K chunk) workgroups of a split run on one XCD,
  // whose L2 then fetches that split's dy slice and W rows once.  The last n_fin workgroups
  // finalise h and g (LoRA).
  constexpr int TS = TW == 64 ? 2 : 4, KS = TS;  // MFMA tiles per wave in tokens and in columns
  constexpr int NQ = TW / 64;                     // float4 of dy staged per thread and step
  const int Kc = a.Kp / 128, ntt = (a.T + 63) / 64, nwt = (a.T + TW - 1) / TW;
  const int nunit = a.nsplit * nwt;  // (token group, row split) units of Kc workgroups each
  const int nmain = (nunit + 7) / 8 * 8 * Kc;
  const int id = blockIdx.x;
  if (id >= nmain) {
    dx_lora_sums(a, id - nmain, gridDim.x - nmain);
    return;  // uniform over the workgroup, before any barrier
  }
  constexpr int D = TW == 64 ? 4 : 3;
  __shared__ u4v sA[2][TW / 16][2][64];                               // [buf][tile][hi/lo][lane]
  __shared__ __attribute__((aligned(16))) _Float16 sW[2][2][128][40];   // [buf][hi/lo][k][n]
  __shared__ float sInv[TW];  // 2^-e (times wunsc) of each token row of the tile
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, li = lane & 15, g = lane >> 4;
  const int wt = TW == 64 ? w >> 2 : w >> 1, wk = TW == 64 ? w & 3 : w & 1;
  // id -> (XCD id % 8, slot id / 8) -> K chunk slot % Kc of unit u = (slot / Kc) * 8 + XCD: the Kc
  // workgroups of a unit run back to back on one XCD and share its dy rows in that L2; unit
  // u = token group * nsplit + split, so an XCD's concurrent units also share weight rows
  const int kc = (id >> 3) % Kc, u = (id >> 3) / Kc * 8 + (id & 7);
  if (u >= nunit) return;  // padding of the unit count to a multiple of 8 (uniform, before any barrier)
  const int sp = u % a.nsplit;
  const int t0 = (u / a.nsplit) * TW;
  const int n0 = sp * a.n_per_split;
  const int nsteps = (min(n0 + a.n_per_split, a.Np) - n0) / 32;
  const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  f4 acc[TS][KS];
#pragma unroll
  for (int i = 0; i < TS; i++)
#pragma unroll
    for (int j = 0; j < KS; j++) acc[i][j] = zero;

  // dy loader: tokens tl + 64 m (m < NQ), float4 q4 (columns ns + 4 q4 .. +3 of the step); wave w
  // covers tokens 16 (w % 4) .. +15 and float4 columns 4 (w / 4) .. +3, so its 64 lanes write the
  // bf16 halves of 32 consecutive A-fragment lanes (512 contiguous bytes: no LDS bank conflicts)
  const int tl = 16 * ((tid >> 6) & 3) + (tid & 15), q4 = 4 * (tid >> 8) + ((tid >> 4) & 3);
  const __amdgpu_buffer_rsrc_t rdy = make_rsrc(a.dy, (uint32_t)a.T * a.N * 4u);
  const uint32_t dy_off = ((uint32_t)(t0 + tl) * a.N + 4 * q4) * 4u;
  const bool dy_vec = (a.N & 3) == 0;
  // W loader (see above)
  const int hh = tid >> 8, rgl = (tid >> 7) & 1, qp = (tid >> 2) & 31, jb = tid & 3;
  const int wp = qp & 7, wgg = qp >> 3;   // rows 2wp, 2wp+1 of row group rgl; k-group wgg
  const int li0 = 2 * wp, FL0 = 16 * wgg + li0;
  const int nloc = rgl * 16 + li0;         // first of the two rows within the step
  constexpr bool KQ = is_kquant(FMT), B8 = byte_codes(FMT);
  const uint32_t wq_bytes = (uint32_t)(a.Np / 16) * Kc * 64 * 16 * (B8 ? 2 : 1);
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.wq, wq_bytes);
  const __amdgpu_buffer_rsrc_t rd = make_rsrc(a.wd, (uint32_t)(a.Np / 16) * Kc * 128);
  const __amdgpu_buffer_rsrc_t re = make_rsrc(a.wsb, KQ ? (uint32_t)(a.Np / 16) * Kc * 32 : 0u);
  uint32_t q_off[2];
#pragma unroll
  for (int r = 0; r < 2; r++) {
    if (!B8)
      q_off[r] = ((((uint32_t)rgl * Kc + kc) * 64 + FL0 + r) * 4 + jb) * 4u;
    else
      q_off[r] = ((((((uint32_t)rgl * Kc + kc) * 2 + (jb >> 1)) * 64 + FL0 + r) * 2 + (jb & 1)) * 2 + hh) * 4u;
  }
  // scales of rows li0, li0+1: adjacent fp16 (Q4_0, Q8_0); for K-quants the two rows' sub-block
  // words (one 16-byte load) and super-block pairs (one 8-byte load)
  const uint32_t d_off = KQ ? (uint32_t)RTQ_WR_INDEX(rgl, kc, Kc, li0, 0) * 2u
                            : (uint32_t)RTQ_WD_INDEX(rgl, kc, Kc, li0, jb) * 2u;
  const uint32_t e_off = (uint32_t)RTQ_WSB_INDEX(rgl, kc >> 1, Kc >> 1, li0) * 4u;
  const uint32_t q_rg = (uint32_t)Kc * 64 * 16 * (B8 ? 2 : 1);  // bytes per row group
  const uint32_t d_rg = (uint32_t)Kc * 128, e_rg = (uint32_t)Kc * 32;

  // 2^e of this thread's dy rows tl + 64 m: e from the largest |dy| of the row over the slices of
  // 256 rows that meet this split (their maxima from rtq_bwd_prep); 1 for a zero row.  All threads
  // reduce the tile's rows: thread (row tid % TW, slices tid / TW + k (512 / TW)), then the partial
  // maxima in LDS (a split may span many slices: 76 for a 19456-row weight).
  float dsc[NQ];
  {
    __shared__ float sRed[512];
    constexpr int PER = 512 / TW;
    const int q0 = n0 / 256, q1 = min((n0 + a.n_per_split + 255) / 256, a.dmq);
    const int tok = tid % TW, t = t0 + tok;
    float mx = 0.0f;
    if (t < a.T) {
#pragma unroll 4
      for (int q = q0 + tid / TW; q < q1; q += PER) mx = fmaxf(mx, a.dymax[(int64_t)q * a.T + t]);
    }
    sRed[tid] = mx;
    __syncthreads();
    if (tid < TW) {
      float m = sRed[tid];
#pragma unroll
      for (int k = 1; k < PER; k++) m = fmaxf(m, sRed[tid + k * TW]);
      int ex = 0;
      (void)frexpf(m, &ex);  // m = f 2^ex, f in [0.5, 1)
      const bool ok = m > 0.0f && m <= 3.0e38f;
      sRed[tid] = ok ? ldexpf(1.0f, 15 - ex) : 1.0f;
      sInv[tid] = (ok ? ldexpf(1.0f, ex - 15) : 1.0f) * a.wunsc;
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < NQ; m++) dsc[m] = sRed[tl + 64 * m];
  }
  // -1 as a run-time value (wsc * wunsc = 1 exactly), so v - hi stays one mixed-precision FMA
  const float neg1 = -(a.wsc * a.wunsc);

  DxSlot<FMT, NQ> sl[D];
  auto issue = [&](DxSlot<FMT, NQ>& S, int step) {
    const int ns = n0 + 32 * min(step, max(nsteps - 1, 0));  // clamped: always a real step
    const uint32_t srg = (uint32_t)(ns >> 4);
#pragma unroll
    for (int m = 0; m < NQ; m++) {
      const uint32_t mo = dy_off + (uint32_t)(64 * m) * a.N * 4u;
      if (dy_vec) {
        S.dy[m] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rdy, mo, (uint32_t)ns * 4u, 0));
      } else {
#pragma unroll
        for (int c = 0; c < 4; c++)
          S.dy[m][c] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rdy, mo + 4u * c, (uint32_t)ns * 4u, 0));
      }
    }
#pragma unroll
    for (int r = 0; r < 2; r++) S.q[r] = __builtin_amdgcn_raw_buffer_load_b32(rq, q_off[r], srg * q_rg, 0);
    if constexpr (KQ) {
      S.k = __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(rd, d_off, srg * d_rg, 0));
      S.e = __builtin_bit_cast(u2v, __builtin_amdgcn_raw_buffer_load_b64(re, e_off, srg * e_rg, 0));
    } else {
      S.d = __builtin_amdgcn_raw_buffer_load_b32(rd, d_off, srg * d_rg, 0);
    }
  };
  // The ragged tail of N (columns >= N of the last step hold the next row's values) is cleared here,
  // where the step's loads are consumed: clearing the load destinations right after issuing them
  // makes the compiler wait for every load in flight, the prefetched steps' included.
  auto stage = [&](const DxSlot<FMT, NQ>& S, int buf, int step) {
    const int nst = n0 + 32 * min(step, max(nsteps - 1, 0));
#pragma unroll
    for (int m = 0; m < NQ; m++) {  // dy: A fragment tile (tl>>4) + 4m, lane (tl&15) + 16*(q4>>1), slots 4*(q4&1) ..
      f4 dv = S.dy[m];
      if (nst + 32 > a.N) {
#pragma unroll
        for (int c = 0; c < 4; c++)
          if (nst + 4 * q4 + c >= a.N) dv[c] = 0.0f;
      }
      const float x0 = dv[0] * dsc[m], x1 = dv[1] * dsc[m], x2 = dv[2] * dsc[m], x3 = dv[3] * dsc[m];
      const half2v h01 = pk_rtz(x0, x1), h23 = pk_rtz(x2, x3);
      // x - hi = dy 2^e - hi exactly (at most 13 significant bits): one mixed-precision FMA each
      const half2v l01 = pk_rtz(fmaf(dv[0], dsc[m], -(float)h01.x), fmaf(dv[1], dsc[m], -(float)h01.y));
      const half2v l23 = pk_rtz(fmaf(dv[2], dsc[m], -(float)h23.x), fmaf(dv[3], dsc[m], -(float)h23.y));
      const u2v hv = {__builtin_bit_cast(uint32_t, h01), __builtin_bit_cast(uint32_t, h23)};
      const u2v lv = {__builtin_bit_cast(uint32_t, l01), __builtin_bit_cast(uint32_t, l23)};
      const int fl = (tl & 15) + 16 * (q4 >> 1);
      reinterpret_cast<u2v*>(&sA[buf][(tl >> 4) + 4 * m][0][fl])[q4 & 1] = hv;
      reinterpret_cast<u2v*>(&sA[buf][(tl >> 4) + 4 * m][1][fl])[q4 & 1] = lv;
    }
    // W: rows 2p, 2p+1 -> f16 hi / lo planes, one 32-bit word (both rows) per column
    uint32_t hw[4], lw[4];
    if constexpr (KQ) {
      float v[2][4];
#pragma unroll
      for (int r = 0; r < 2; r++) {
        float d, m;
        dq_params<FMT>(0u, comp(S.k, 2 * r + (jb >> 1)), r ? S.e.y : S.e.x, jb, hh, d, m);
        d *= a.wsc;  // exact (a power of two; 1 unless a scale is huge)
        m *= a.wsc;
        const uint32_t u = B8 ? S.q[r] ^ 0x80808080u : (hh ? (S.q[r] >> 4) : S.q[r]) & 0x0f0f0f0fu;
#pragma unroll
        for (int e = 0; e < 4; e++) v[r][e] = fmaf((float)((u >> (8 * e)) & 0xffu), d, m);  // rounded once, as ggml
      }
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const half2v h = pk_rtz(v[0][e], v[1][e]);
        hw[e] = __builtin_bit_cast(uint32_t, h);
        lw[e] = __builtin_bit_cast(uint32_t, pk_rtz(fmaf((float)h.x, neg1, v[0][e]), fmaf((float)h.y, neg1, v[1][e])));
      }
    } else {
      // codes as exact f16 pairs (1024 + u of row 2p, of row 2p+1): bytes interleaved by row, then
      // each pair of bytes widened with 0x64, the high byte of 1024.0; c = that - (1024 + offset)
      const uint32_t u0 = B8 ? S.q[0] ^ 0x80808080u : (hh ? (S.q[0] >> 4) : S.q[0]) & 0x0f0f0f0fu;
      const uint32_t u1 = B8 ? S.q[1] ^ 0x80808080u : (hh ? (S.q[1] >> 4) : S.q[1]) & 0x0f0f0f0fu;
      const uint32_t i01 = __builtin_amdgcn_perm(u1, u0, 0x05010400u), i23 = __builtin_amdgcn_perm(u1, u0, 0x07030602u);
      half2v dp = __builtin_bit_cast(half2v, S.d);  // fp16 scales of rows 2p, 2p+1
      dp = dp * half2v{(_Float16)a.wsc, (_Float16)a.wsc};  // exact, as for the K-quants
      constexpr _Float16 OFF = B8 ? (_Float16)1152.0f : (_Float16)1032.0f;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const uint32_t src = e < 2 ? i01 : i23;
        const half2v c = sub_h2((e & 1) ? bytes23_to_h2(src) : bytes01_to_h2(src), OFF);
        const half2v h = dp * c;                                // f16 product, rounded
        const half2v l = __builtin_elementwise_fma(dp, c, -h);  // its exact residual
        hw[e] = __builtin_bit_cast(uint32_t, h);
        lw[e] = __builtin_bit_cast(uint32_t, l);
      }
    }
    const int kb = 32 * jb + 16 * hh + 4 * wgg;
    const int ns = nloc ^ (8 * jb);  // swizzled row (pair start stays even)
#pragma unroll
    for (int e = 0; e < 4; e++) {
      *reinterpret_cast<uint32_t*>(&sW[buf][0][kb + e][ns]) = hw[e];
      *reinterpret_cast<uint32_t*>(&sW[buf][1][kb + e][ns]) = lw[e];
    }
  };
  // the wave's operand fragments of one step: A (dy) hi / lo of its two token tiles, B (W) hi / lo
  // of its two column tiles
  struct Frags {
    half8 a[TS][2], b[KS][2];
  };
  auto load_frags = [&](int buf, Frags& F) {
#pragma unroll
    for (int ts = 0; ts < TS; ts++) {
      F.a[ts][0] = __builtin_bit_cast(half8, sA[buf][wt * TS + ts][0][lane]);
      F.a[ts][1] = __builtin_bit_cast(half8, sA[buf][wt * TS + ts][1][lane]);
    }
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
      // column kl lies in block kl / 32, whose rows are swizzled by 8 (kl / 32)
      const int kl = wk * 16 * KS + ks * 16 + li, jbk = (wk * 16 * KS + ks * 16) >> 5;
      F.b[ks][0] = *reinterpret_cast<const half8*>(&sW[buf][0][kl][8 * (g ^ jbk)]);
      F.b[ks][1] = *reinterpret_cast<const half8*>(&sW[buf][1][kl][8 * (g ^ jbk)]);
    }
  };
  auto compute = [&](const Frags& F) {
#pragma unroll
    for (int ts = 0; ts < TS; ts++)
#pragma unroll
      for (int ks = 0; ks < KS; ks++) {
        acc[ts][ks] = mfma_f16(F.a[ts][0], F.b[ks][0], acc[ts][ks]);
        acc[ts][ks] = mfma_f16(F.a[ts][1], F.b[ks][0], acc[ts][ks]);
        acc[ts][ks] = mfma_f16(F.a[ts][0], F.b[ks][1], acc[ts][ks]);
      }
  };
  // Step s: one barrier (buffer s & 1 is staged by all waves, buffer (s + 1) & 1 is free: every
  // wave has finished step s - 1's reads), then step s's fragments are read from LDS, step s + 1 is
  // staged while those reads complete (LDS operations complete in order: reads issued first), and
  // step s's MFMAs run under the staging's tail.  Loads run D - 1 steps ahead of the MFMAs.
#pragma unroll
  for (int s0 = 0; s0 < D - 1; s0++) issue(sl[s0], s0);
  if (nsteps > 0) stage(sl[0], 0, 0);
  // one step of the loop; `full`: a step of a complete group of D (no guards, one basic block, so
  // the scheduler can interleave the MFMAs with the staging arithmetic; staging past the last step
  // only writes the unused buffer)
  auto step_body = [&](int s0, int step, bool full) {
    issue(sl[(s0 + D - 1) % D], step + D - 1);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    Frags F;
    if (full || step < nsteps) load_frags(step & 1, F);
    if (full || step + 1 < nsteps) stage(sl[(s0 + 1) % D], (step + 1) & 1, step + 1);
    if (full || step < nsteps) compute(F);
    if (full) {
#pragma unroll
      for (int m = 0; m < 3 * TS * KS; m++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);              // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, TW == 64 ? 4 : 2, 0);  // VALU
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  const int nfull = nsteps / D * D;
  for (int st0 = 0; st0 < nfull; st0 += D) {
#pragma unroll
    for (int s0 = 0; s0 < D; s0++) step_body(s0, st0 + s0, true);
  }
  if (nfull < nsteps) {
#pragma unroll
    for (int s0 = 0; s0 < D; s0++) step_body(s0, nfull + s0, false);
  }
  // rows back to dy's scale (and W's): element i of acc[ts][ks] is tile row TW == 64 ? 32wt + 16ts + 4g + i
  // : 64wt + 16ts + 4g + i (sInv was written before the loop's first barrier)
#pragma unroll
  for (int ts = 0; ts < TS; ts++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float sv = sInv[(TW == 64 ? 32 : 64) * wt + 16 * ts + 4 * g + i];
#pragma unroll
      for (int ks = 0; ks < KS; ks++) acc[ts][ks][i] *= sv;
    }
  // partial tile of this split in fragment order: part[sp][tile][wave][q][lane] (float4 each),
  // tile = 64-token tile * Kc + K chunk, wave = 4 wt' + wk', q = 2 ts' + ks' in the TW = 64 layout:
  // element i is row 64 tile + 32wt' + 16ts' + 4g + i, column 128kc + 32wk' + 16ks' + li.  Each
  // 16-byte store of a wave writes 1 KB contiguously.
  if (TW == 64) {
    f4* out = reinterpret_cast<f4*>(a.part) + ((((int64_t)sp * ntt + (t0 >> 6)) * Kc + kc) * 8 + w) * 256 + lane;
#pragma unroll
    for (int ts = 0; ts < 2; ts++)
#pragma unroll
      for (int ks = 0; ks < 2; ks++) out[(ts * 2 + ks) * 64] = acc[ts][ks];
  } else {
    const int tt64 = (t0 >> 6) + wt;  // this wave's 64 tokens form one 64-token tile
    if (tt64 < ntt) {
      f4* out = reinterpret_cast<f4*>(a.part) + (((int64_t)sp * ntt + tt64) * Kc + kc) * 8 * 256 + lane;
#pragma unroll
      for (int ts = 0; ts < 4; ts++)
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
          const int wo = (ts >> 1) * 4 + 2 * wk + (ks >> 1), qo = (ts & 1) * 2 + (ks & 1);
          out[(wo * 4 + qo) * 64] = acc[ts][ks];
        }
    }
  }
}

// ============================================================== dx = dy . W for T = 1
// One token: dx[k] = sum_n dy[n] W[n][k] with f32 FMAs, no MFMA.  Workgroup (K chunk kc, row split
// sp) of four waves; wave w takes the row groups rg0 + w, rg0 + w + 4, .. of the split through a
// D-deep register ring.  Lane (row li, k-group g) holds, per row group, the codes of row
// n = 16 rg + li for the 32 columns {32j + 4g .. + 3, 32j + 16 + 4g .. + 3} (j < 4) of the chunk (the
// device layout), turns them into exact f16 values (the code less its offset: Q4_0 u - 8, Q8_0 /
// Q6_K q, Q4_K u) and adds c * value into its 32 column sums by mixed-precision FMA, c = dy[n] times
// the row's scale for that block (Q4_K: d sc; its - dmin m part enters as dy[n] dmin m summed per
// block and subtracted once; Q6_K: d sc of each 16-element half).  The 16 rows of a k-group (one
// DPP row of lanes) are added by four DPP steps, the four waves in wave order through LDS, and the
// workgroup writes part[sp][0][128 kc ..] row-major (rtq_bwd_finish adds the splits in order).
template <int FMT>
struct Dxv1Slot {
  u4v q[byte_codes(FMT) ? 2 : 1];  // codes (nibble layout, or byte layout in two parts)
  u2v d;                           // row li, blocks 0..3: fp16 scales / K-quant sub-block words
  uint32_t e;                      // K-quants: the row's super-block (d, dmin)
  float dy;                        // dy of the row
};

template <int FMT>
__device__ __forceinline__ void dxv1_tile(const DxArgs& a) {
  constexpr bool KQ = is_kquant(FMT), B8 = byte_codes(FMT);
  constexpr int D = RTQ_DXV1_D;
  const int Kc = a.Kp / 128, ngroups = a.Np / 16;
  const int nmain = Kc * a.nsplit;
  const int id = blockIdx.x;
  if (id >= nmain) {
    dx_lora_sums(a, id - nmain, gridDim.x - nmain);
    return;  // uniform over the workgroup, before any barrier
  }
  __shared__ float red[4][128];
  const int tid = threadIdx.x, lane = tid & 63, li = lane & 15, g = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kc = id % Kc, sp = id / Kc;
  const int rps = a.n_per_split / 16;  // row groups per split
  const int rg0 = sp * rps, rg1 = min(rg0 + rps, ngroups);
  const int nit = rg1 - rg0 > w ? (rg1 - rg0 - w + 3) / 4 : 0;
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.wq, (uint32_t)ngroups * Kc * 1024u * (B8 ? 2u : 1u));
  const __amdgpu_buffer_rsrc_t rd = make_rsrc(a.wdr, (uint32_t)ngroups * Kc * 128u);
  const __amdgpu_buffer_rsrc_t re = make_rsrc(a.wsb, KQ ? (uint32_t)ngroups * (Kc >> 1) * 64u : 0u);
  const __amdgpu_buffer_rsrc_t rdy = make_rsrc(a.dy, (uint32_t)a.N * 4u);  // rows >= N read zero
  auto issue = [&](Dxv1Slot<FMT>& S, int it) {
    const uint32_t rg = (uint32_t)(rg0 + w + 4 * min(it, max(nit - 1, 0))), base = rg * Kc + kc;  // clamped
    if (B8) {
      S.q[0] = __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(rq, lane * 16u, base * 2048u, 0));
      S.q[B8 ? 1 : 0] = __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(rq, lane * 16u, base * 2048u + 1024u, 0));
    } else {
      S.q[0] = __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(rq, lane * 16u, base * 1024u, 0));
    }
    S.d = __builtin_bit_cast(u2v, __builtin_amdgcn_raw_buffer_load_b64(rd, li * 8u, base * 128u, 0));
    if (KQ) S.e = __builtin_amdgcn_raw_buffer_load_b32(re, li * 4u, (rg * (Kc >> 1) + (kc >> 1)) * 64u, 0);
    S.dy = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rdy, li * 4u, rg * 64u, 0));
  };
  float acc[4][8], bias[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    bias[j] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) acc[j][e] = 0.0f;
  }
  auto compute = [&](const Dxv1Slot<FMT>& S) {
    // K-quants: dy times the row's super-block scales, once per item (then times each block's
    // integer scale)
    const float dyd = KQ ? S.dy * h2f((uint16_t)(S.e & 0xffffu)) : 0.0f;
    const float dym = FMT == FMT_Q4_K ? S.dy * h2f((uint16_t)(S.e >> 16)) : 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t wv = hcomp(S.d, j);
      half8 f;
      float c, c2 = 0.0f;  // c2: Q6_K, the second half's factor
      if constexpr (FMT == FMT_Q4_0 || FMT == FMT_Q8_0) {
        c = S.dy * h2f((uint16_t)wv);
        if (FMT == FMT_Q4_0) {
          f = q4_0_frag<8>(comp(S.q[0], j));
        } else {
          const u4v& qq = S.q[j >> 1];
          f = (j & 1) ? q8_frag(qq.z, qq.w) : q8_frag(qq.x, qq.y);
        }
      } else if constexpr (FMT == FMT_Q4_K) {  // value d sc u - dmin m (sc, m < 64: whole bytes)
        c = dyd * (float)(wv & 0xffu);
        bias[j] = fmaf(dym, (float)((wv >> 8) & 0xffu), bias[j]);
        f = q4_0_frag<0>(comp(S.q[0], j));
      } else {  // Q6_K: value d sc q, sc per 16 elements (low byte: elements 0..15 of the block)
        c = dyd * (float)(int)(int8_t)(wv & 0xffu);
        c2 = dyd * (float)(int)(int8_t)((wv >> 8) & 0xffu);
        const u4v& qq = S.q[j >> 1];
        f = (j & 1) ? q8_frag(qq.z, qq.w) : q8_frag(qq.x, qq.y);
      }
#pragma unroll
      for (int e = 0; e < 8; e++) acc[j][e] = fmaf(FMT == FMT_Q6_K && e >= 4 ? c2 : c, (float)f[e], acc[j][e]);
    }
  };
  Dxv1Slot<FMT> sl[D];
#pragma unroll
  for (int s0 = 0; s0 < D - 1; s0++) issue(sl[s0], s0);
  for (int it0 = 0; it0 < nit; it0 += D) {
#pragma unroll
    for (int s0 = 0; s0 < D; s0++) {
      issue(sl[(s0 + D - 1) % D], it0 + s0 + D - 1);
      __builtin_amdgcn_sched_barrier(0);
      if (it0 + s0 < nit) compute(sl[s0]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // the 16 rows of each k-group: lanes i ^ 1, the quad, the other quad of the eight, the other eight
#pragma unroll
  for (int j = 0; j < 4; j++) {
    if (FMT == FMT_Q4_K) {
#pragma unroll
      for (int e = 0; e < 8; e++) acc[j][e] -= bias[j];
    }
#pragma unroll
    for (int e = 0; e < 8; e++) {
      float v = acc[j][e];
      v += dpp_f<0xB1>(v);
      v += dpp_f<0x4E>(v);
      v += dpp_f<0x141>(v);
      v += dpp_f<0x140>(v);
      acc[j][e] = v;
    }
  }
  if (li == 0) {  // lane (0, g): columns 32j + 4g + e (e < 4) and 32j + 16 + 4g + e - 4 (e >= 4)
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int e = 0; e < 8; e++) red[w][32 * j + (e < 4 ? 4 * g + e : 16 + 4 * g + e - 4)] = acc[j][e];
  }
  __syncthreads();
  if (tid < 128) {
    const int col = kc * 128 + tid;
    const float v = ((red[0][tid] + red[1][tid]) + red[2][tid]) + red[3][tid];
    if (col < a.K) a.part[(int64_t)sp * a.K + col] = v;  // (no f16 weight values: no pre-scaling to undo)
  }
}

// ============================================================== dx = dy . W for T <= 16
// Same arithmetic as dx_tile with one 16-token tile: workgroup of 4 waves, tile 16 tokens x 128
// columns (wave w: the 32 columns of block w), 32 rows per step, many row splits (a GEMV-shaped
// product needs them to fill the GPU).  Each thread stages both halves of its W words, and the
// partials are written row-major for the real tokens only: part[split][t][k].  f16 hi / lo operands
// as in dx_tile; dy's scale 2^e per token from the largest |dy| over this split's rows, found by the
// workgroup itself (wave w: tokens w, w + 4, ..), while the first steps' loads are in flight.
template <int FMT>
struct Dx16Slot {
  float2 dy;          // rows 2p, 2p+1 of the step, token tid / 16
  uint32_t q[2][2];   // [row][half] code words (nibble formats: both halves in q[r][0])
  uint32_t d;         // fp16 scales of the two rows (Q4_0, Q8_0)
  u4v k;              // sub-block scale words of the two rows (K-quants, as DxSlot)
  u2v e;              // super-block scales of the two rows (K-quants)
};

template <int FMT>
__device__ __forceinline__ void dx16_tile(const DxArgs& a) {
  const int Kc = a.Kp / 128;
  const int nmain = Kc * a.nsplit;
  const int id = blockIdx.x;
  if (id >= nmain) {
    dx_lora_sums(a, id - nmain, gridDim.x - nmain);
    return;  // uniform over the workgroup, before any barrier
  }
  constexpr bool KQ = is_kquant(FMT), B8 = byte_codes(FMT);
  constexpr int D = RTQ_DX16_D;
  __shared__ u4v sA[2][2][64];                                          // [buf][hi/lo][lane]
  __shared__ __attribute__((aligned(16))) _Float16 sW[2][2][128][40];   // [buf][hi/lo][k][n]
  __shared__ float sSc[16], sInv[16];  // 2^e of each token row, 2^-e (times wunsc)
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, li = lane & 15, g = lane >> 4;
  // id -> (split, K chunk), XCD-aware as in dx_tile
  int sp, kc;
  if ((a.nsplit & 7) == 0) {
    const int grp = id / (8 * Kc), rem = id % (8 * Kc);
    sp = grp * 8 + rem % 8;
    kc = rem / 8;
  } else {
    sp = id / Kc;
    kc = id % Kc;
  }
  const int n0 = sp * a.n_per_split;
  const int nsteps = (min(n0 + a.n_per_split, a.Np) - n0) / 32;
  const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  f4 acc[2] = {zero, zero};

  // dy loader: token tl = tid >> 4, rows 2pp, 2pp+1 of the step (tokens >= T read zero)
  const int tl = tid >> 4, pp = tid & 15;
  const __amdgpu_buffer_rsrc_t rdy = make_rsrc(a.dy, (uint32_t)a.T * a.N * 4u);
  const uint32_t dy_off = ((uint32_t)tl * a.N + 2 * pp) * 4u;
  const bool dy_vec = (a.N & 1) == 0;
  // W loader: row group rgl, rows 2wp, 2wp+1, k-group wgg, block jb (both halves)
  const int rgl = tid >> 7, qp = (tid >> 2) & 31, jb = tid & 3;
  const int wp = qp & 7, wgg = qp >> 3;
  const int li0 = 2 * wp, FL0 = 16 * wgg + li0;
  const int nloc = rgl * 16 + li0;
  const uint32_t wq_bytes = (uint32_t)(a.Np / 16) * Kc * 64 * 16 * (B8 ? 2 : 1);
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.wq, wq_bytes);
  const __amdgpu_buffer_rsrc_t rd = make_rsrc(a.wd, (uint32_t)(a.Np / 16) * Kc * 128);
  const __amdgpu_buffer_rsrc_t re = make_rsrc(a.wsb, KQ ? (uint32_t)(a.Np / 16) * Kc * 32 : 0u);
  uint32_t q_off[2];
#pragma unroll
  for (int r = 0; r < 2; r++) {
    if (!B8)
      q_off[r] = ((((uint32_t)rgl * Kc + kc) * 64 + FL0 + r) * 4 + jb) * 4u;
    else
      q_off[r] = (((((uint32_t)rgl * Kc + kc) * 2 + (jb >> 1)) * 64 + FL0 + r) * 2 + (jb & 1)) * 8u;
  }
  const uint32_t d_off = KQ ? (uint32_t)RTQ_WR_INDEX(rgl, kc, Kc, li0, 0) * 2u
                            : (uint32_t)RTQ_WD_INDEX(rgl, kc, Kc, li0, jb) * 2u;
  const uint32_t e_off = (uint32_t)RTQ_WSB_INDEX(rgl, kc >> 1, Kc >> 1, li0) * 4u;
  const uint32_t q_rg = (uint32_t)Kc * 64 * 16 * (B8 ? 2 : 1);
  const uint32_t d_rg = (uint32_t)Kc * 128, e_rg = (uint32_t)Kc * 32;
  // -1 as a run-time value (wsc * wunsc = 1 exactly), so v - hi stays one mixed-precision FMA
  const float neg1 = -(a.wsc * a.wunsc);

  Dx16Slot<FMT> sl[D];
  auto issue = [&](Dx16Slot<FMT>& S, int step) {
    const int ns = n0 + 32 * min(step, max(nsteps - 1, 0));  // clamped: always a real step
    const uint32_t srg = (uint32_t)(ns >> 4);
    if (dy_vec) {
      S.dy = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(rdy, dy_off, (uint32_t)ns * 4u, 0));
    } else {
      S.dy.x = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rdy, dy_off, (uint32_t)ns * 4u, 0));
      S.dy.y = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rdy, dy_off + 4u, (uint32_t)ns * 4u, 0));
    }
    if (ns + 32 > a.N) {  // ragged tail of N: columns >= N hold the next token's values
      if (ns + 2 * pp >= a.N) S.dy.x = 0.0f;
      if (ns + 2 * pp + 1 >= a.N) S.dy.y = 0.0f;
    }
#pragma unroll
    for (int r = 0; r < 2; r++) {
      if (B8) {
        const u2v v = __builtin_bit_cast(u2v, __builtin_amdgcn_raw_buffer_load_b64(rq, q_off[r], srg * q_rg, 0));
        S.q[r][0] = v.x;
        S.q[r][1] = v.y;
      } else {
        S.q[r][0] = __builtin_amdgcn_raw_buffer_load_b32(rq, q_off[r], srg * q_rg, 0);
      }
    }
    if constexpr (KQ) {
      S.k = __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(rd, d_off, srg * d_rg, 0));
      S.e = __builtin_bit_cast(u2v, __builtin_amdgcn_raw_buffer_load_b64(re, e_off, srg * e_rg, 0));
    } else {
      S.d = __builtin_amdgcn_raw_buffer_load_b32(rd, d_off, srg * d_rg, 0);
    }
  };
  float dsc = 1.0f;  // 2^e of this thread's token tl
  auto stage_compute = [&](const Dx16Slot<FMT>& S, int buf) {
    {  // dy 2^e -> f16 hi / lo: A fragment lane tl + 16 (pp >> 2), slots 2 (pp & 3), +1
      const half2v h = pk_rtz(S.dy.x * dsc, S.dy.y * dsc);
      // dy 2^e - hi exactly (at most 13 significant bits): one mixed-precision FMA each
      const half2v l = pk_rtz(fmaf(S.dy.x, dsc, -(float)h.x), fmaf(S.dy.y, dsc, -(float)h.y));
      const int fl = tl + 16 * (pp >> 2);
      reinterpret_cast<uint32_t*>(&sA[buf][0][fl])[pp & 3] = __builtin_bit_cast(uint32_t, h);
      reinterpret_cast<uint32_t*>(&sA[buf][1][fl])[pp & 3] = __builtin_bit_cast(uint32_t, l);
    }
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {  // W: rows li0, li0+1, half hh -> f16 hi / lo (as dx_tile)
      uint32_t hw[4], lw[4];
      if constexpr (KQ) {
        float v[2][4];
#pragma unroll
        for (int r = 0; r < 2; r++) {
          float d, m;
          dq_params<FMT>(0u, comp(S.k, 2 * r + (jb >> 1)), r ? S.e.y : S.e.x, jb, hh, d, m);
          d *= a.wsc;  // exact (a power of two; 1 unless a scale is huge)
          m *= a.wsc;
          const uint32_t u = B8 ? S.q[r][hh] ^ 0x80808080u : (hh ? (S.q[r][0] >> 4) : S.q[r][0]) & 0x0f0f0f0fu;
#pragma unroll
          for (int e = 0; e < 4; e++) v[r][e] = fmaf((float)((u >> (8 * e)) & 0xffu), d, m);  // rounded once, as ggml
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const half2v h = pk_rtz(v[0][e], v[1][e]);
          hw[e] = __builtin_bit_cast(uint32_t, h);
          lw[e] = __builtin_bit_cast(uint32_t, pk_rtz(fmaf((float)h.x, neg1, v[0][e]), fmaf((float)h.y, neg1, v[1][e])));
        }
      } else {
        // codes as exact f16 pairs (1024 + u of row 2p, of row 2p+1), c = that - (1024 + offset);
        // hi = f16(d c), lo its exact residual
        const uint32_t u0 = B8 ? S.q[0][hh] ^ 0x80808080u : (hh ? (S.q[0][0] >> 4) : S.q[0][0]) & 0x0f0f0f0fu;
        const uint32_t u1 = B8 ? S.q[1][hh] ^ 0x80808080u : (hh ? (S.q[1][0] >> 4) : S.q[1][0]) & 0x0f0f0f0fu;
        const uint32_t i01 = __builtin_amdgcn_perm(u1, u0, 0x05010400u), i23 = __builtin_amdgcn_perm(u1, u0, 0x07030602u);
        half2v dp = __builtin_bit_cast(half2v, S.d);  // fp16 scales of rows 2p, 2p+1
        dp = dp * half2v{(_Float16)a.wsc, (_Float16)a.wsc};  // exact, as for the K-quants
        constexpr _Float16 OFF = B8 ? (_Float16)1152.0f : (_Float16)1032.0f;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const uint32_t src = e < 2 ? i01 : i23;
          const half2v c = sub_h2((e & 1) ? bytes23_to_h2(src) : bytes01_to_h2(src), OFF);
          const half2v h = dp * c;
          const half2v l = __builtin_elementwise_fma(dp, c, -h);
          hw[e] = __builtin_bit_cast(uint32_t, h);
          lw[e] = __builtin_bit_cast(uint32_t, l);
        }
      }
      const int kb = 32 * jb + 16 * hh + 4 * wgg;
      const int nsw = nloc ^ (8 * jb);
#pragma unroll
      for (int e = 0; e < 4; e++) {
        *reinterpret_cast<uint32_t*>(&sW[buf][0][kb + e][nsw]) = hw[e];
        *reinterpret_cast<uint32_t*>(&sW[buf][1][kb + e][nsw]) = lw[e];
      }
    }
    __syncthreads();
    const half8 ah = __builtin_bit_cast(half8, sA[buf][0][lane]);
    const half8 al = __builtin_bit_cast(half8, sA[buf][1][lane]);
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
      const int kl = w * 32 + ks * 16 + li;  // column kl lies in block w: rows swizzled by 8 w
      const half8 bh = *reinterpret_cast<const half8*>(&sW[buf][0][kl][8 * (g ^ w)]);
      const half8 bl = *reinterpret_cast<const half8*>(&sW[buf][1][kl][8 * (g ^ w)]);
      acc[ks] = mfma_f16(ah, bh, acc[ks]);
      acc[ks] = mfma_f16(al, bh, acc[ks]);
      acc[ks] = mfma_f16(ah, bl, acc[ks]);
    }
  };
#pragma unroll
  for (int s0 = 0; s0 < D - 1; s0++) issue(sl[s0], s0);
  {  // the tokens' scales while those loads are in flight: the 16 threads of token tl (the dy
     // loader's) scan its rows of the split together, 64 rows per step (a float4 each, or four
     // floats where N % 4 != 0), RTQ_DX16_SCAN steps' loads in flight, then a max over the 16
    const int r1 = min(n0 + a.n_per_split, a.N);
    float mx = 0.0f;
    if (tl < a.T) {
      const float* row = a.dy + (int64_t)tl * a.N;
      const bool v4 = (a.N & 3) == 0 && (reinterpret_cast<uintptr_t>(a.dy) & 15) == 0;  // uniform: 16-byte aligned rows (n0 % 32 == 0)
      for (int nb = n0 + 4 * pp; nb < r1; nb += 64 * RTQ_DX16_SCAN) {
        f4 v[RTQ_DX16_SCAN];
#pragma unroll
        for (int u = 0; u < RTQ_DX16_SCAN; u++) {
          const int n = nb + 64 * u;
          if (v4 && n + 4 <= r1) {
            v[u] = *reinterpret_cast<const f4*>(row + n);
          } else {
#pragma unroll
            for (int e = 0; e < 4; e++) v[u][e] = n + e < r1 ? row[n + e] : 0.0f;
          }
        }
#pragma unroll
        for (int u = 0; u < RTQ_DX16_SCAN; u++)
#pragma unroll
          for (int e = 0; e < 4; e++) mx = fmaxf(mx, fabsf(v[u][e]));
      }
    }
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) mx = fmaxf(mx, __shfl_xor(mx, m));  // the token's 16 lanes
    if (pp == 0 && tl < a.T) {
      int ex = 0;
      (void)frexpf(mx, &ex);  // mx = f 2^ex, f in [0.5, 1): mx 2^(15 - ex) in [2^14, 2^15)
      const bool ok = mx > 0.0f && mx <= 3.0e38f;
      sSc[tl] = ok ? ldexpf(1.0f, 15 - ex) : 1.0f;
      sInv[tl] = (ok ? ldexpf(1.0f, ex - 15) : 1.0f) * a.wunsc;
    }
    __syncthreads();
    if (tl < a.T) dsc = sSc[tl];
  }
  for (int st0 = 0; st0 < nsteps; st0 += D) {
#pragma unroll
    for (int s0 = 0; s0 < D; s0++) {
      issue(sl[(s0 + D - 1) % D], st0 + s0 + D - 1);
      __builtin_amdgcn_sched_barrier(0);
      if (st0 + s0 < nsteps) stage_compute(sl[s0], (st0 + s0) & 1);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // lane holds tokens 4g .. 4g+3 of column 128 kc + 32 w + 16 ks + li, at dy's scale 2^e (and W's)
#pragma unroll
  for (int ks = 0; ks < 2; ks++) {
    const int col = kc * 128 + w * 32 + ks * 16 + li;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int t = 4 * g + e;
      if (t < a.T && col < a.K) a.part[((int64_t)sp * a.T + t) * a.K + col] = acc[ks][e] * sInv[t];
    }
  }
}

// ============================================================== dx = dy . W, 32-token tiles
// dx_tile's arithmetic and partial layout on four-wave workgroups of 32 tokens x 128 columns (wave
// w: columns 32 w .. 32 w + 31, both 16-token MFMA tiles): twice the workgroups of the 64-token
// tiles for the same row splits, so that short token ranges (the training step's 512) give the CUs
// two independent workgroups each.  Each thread stages both halves of its W words (as rtq_dx16_*)
// and one float4 of dy; the partials keep the 64-token fragment order (this workgroup's waves are
// waves 4 wt + wk of the 64-token tile, wt = (t0 % 64) / 32), so rtq_bwd_finish reads them alike.
template <int FMT>
__device__ __forceinline__ void dx32_tile(const DxArgs& a) {
  const int Kc = a.Kp / 128, ntt = (a.T + 63) / 64, nwt = (a.T + 31) / 32;
  const int nunit = a.nsplit * nwt;
  const int nmain = (nunit + 7) / 8 * 8 * Kc;
  const int id = blockIdx.x;
  if (id >= nmain) {
    dx_lora_sums(a, id - nmain, gridDim.x - nmain);
    return;  // uniform over the workgroup, before any barrier
  }
  constexpr bool KQ = is_kquant(FMT), B8 = byte_codes(FMT);
  constexpr int D = 4;
  __shared__ u4v sA[2][2][2][64];                                       // [buf][token tile][hi/lo][lane]
  __shared__ __attribute__((aligned(16))) _Float16 sW[2][2][128][40];   // [buf][hi/lo][k][n]
  __shared__ float sInv[32];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, li = lane & 15, g = lane >> 4;
  // id -> unit and K chunk as dx_tile (the Kc workgroups of a unit back to back on one XCD)
  const int kc = (id >> 3) % Kc, u = (id >> 3) / Kc * 8 + (id & 7);
  if (u >= nunit) return;  // padding of the unit count to a multiple of 8 (uniform, before any barrier)
  const int sp = u % a.nsplit;
  const int t0 = (u / a.nsplit) * 32;
  const int n0 = sp * a.n_per_split;
  const int nsteps = (min(n0 + a.n_per_split, a.Np) - n0) / 32;
  const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  f4 acc[2][2] = {{zero, zero}, {zero, zero}};

  // dy loader: token tl, float4 q4 (rows ns + 4 q4 .. +3 of the step); a wave covers 16 tokens and
  // four float4 columns, so its lanes write 32 consecutive A-fragment lanes' halves
  const int tl = 16 * (w & 1) + (tid & 15), q4 = 4 * (w >> 1) + ((tid >> 4) & 3);
  const __amdgpu_buffer_rsrc_t rdy = make_rsrc(a.dy, (uint32_t)a.T * a.N * 4u);
  const uint32_t dy_off = ((uint32_t)(t0 + tl) * a.N + 4 * q4) * 4u;
  const bool dy_vec = (a.N & 3) == 0;
  // W loader (as rtq_dx16_*): row group rgl, rows 2wp, 2wp+1, k-group wgg, block jb, both halves
  const int rgl = tid >> 7, qp = (tid >> 2) & 31, jb = tid & 3;
  const int wp = qp & 7, wgg = qp >> 3;
  const int li0 = 2 * wp, FL0 = 16 * wgg + li0;
  const int nloc = rgl * 16 + li0;
  const uint32_t wq_bytes = (uint32_t)(a.Np / 16) * Kc * 64 * 16 * (B8 ? 2 : 1);
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.wq, wq_bytes);
  const __amdgpu_buffer_rsrc_t rd = make_rsrc(a.wd, (uint32_t)(a.Np / 16) * Kc * 128);
  const __amdgpu_buffer_rsrc_t re = make_rsrc(a.wsb, KQ ? (uint32_t)(a.Np / 16) * Kc * 32 : 0u);
  uint32_t q_off[2];
#pragma unroll
  for (int r = 0; r < 2; r++) {
    if (!B8)
      q_off[r] = ((((uint32_t)rgl * Kc + kc) * 64 + FL0 + r) * 4 + jb) * 4u;
    else
      q_off[r] = (((((uint32_t)rgl * Kc + kc) * 2 + (jb >> 1)) * 64 + FL0 + r) * 2 + (jb & 1)) * 8u;
  }
  const uint32_t d_off = KQ ? (uint32_t)RTQ_WR_INDEX(rgl, kc, Kc, li0, 0) * 2u
                            : (uint32_t)RTQ_WD_INDEX(rgl, kc, Kc, li0, jb) * 2u;
  const uint32_t e_off = (uint32_t)RTQ_WSB_INDEX(rgl, kc >> 1, Kc >> 1, li0) * 4u;
  const uint32_t q_rg = (uint32_t)Kc * 64 * 16 * (B8 ? 2 : 1);
  const uint32_t d_rg = (uint32_t)Kc * 128, e_rg = (uint32_t)Kc * 32;

  // 2^e of this thread's dy row from the row maxima of the 256-row slices meeting this split
  // (rtq_bwd_prep), reduced by all threads: thread (row tid % 32, slices tid / 32 + 8 k)
  float dsc;
  {
    __shared__ float sRed[256];
    const int q0 = n0 / 256, q1 = min((n0 + a.n_per_split + 255) / 256, a.dmq);
    const int tok = tid % 32, t = t0 + tok;
    float mx = 0.0f;
    if (t < a.T) {
#pragma unroll 4
      for (int qq = q0 + tid / 32; qq < q1; qq += 8) mx = fmaxf(mx, a.dymax[(int64_t)qq * a.T + t]);
    }
    sRed[tid] = mx;
    __syncthreads();
    if (tid < 32) {
      float m = sRed[tid];
#pragma unroll
      for (int k = 1; k < 8; k++) m = fmaxf(m, sRed[tid + k * 32]);
      int ex = 0;
      (void)frexpf(m, &ex);  // m = f 2^ex, f in [0.5, 1)
      const bool ok = m > 0.0f && m <= 3.0e38f;
      sRed[tid] = ok ? ldexpf(1.0f, 15 - ex) : 1.0f;
      sInv[tid] = (ok ? ldexpf(1.0f, ex - 15) : 1.0f) * a.wunsc;
    }
    __syncthreads();
    dsc = sRed[tl];
  }
  const float neg1 = -(a.wsc * a.wunsc);

  Dx16Slot<FMT> sl[D];  // (its float2 dy unused here: a float4 in dy4)
  f4 dy4[D];
  auto issue = [&](int slot, int step) {
    Dx16Slot<FMT>& S = sl[slot];
    const int ns = n0 + 32 * min(step, max(nsteps - 1, 0));  // clamped: always a real step
    const uint32_t srg = (uint32_t)(ns >> 4);
    if (dy_vec) {
      dy4[slot] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rdy, dy_off, (uint32_t)ns * 4u, 0));
    } else {
#pragma unroll
      for (int c = 0; c < 4; c++)
        dy4[slot][c] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rdy, dy_off + 4u * c, (uint32_t)ns * 4u, 0));
    }
#pragma unroll
    for (int r = 0; r < 2; r++) {
      if (B8) {
        const u2v v = __builtin_bit_cast(u2v, __builtin_amdgcn_raw_buffer_load_b64(rq, q_off[r], srg * q_rg, 0));
        S.q[r][0] = v.x;
        S.q[r][1] = v.y;
      } else {
        S.q[r][0] = __builtin_amdgcn_raw_buffer_load_b32(rq, q_off[r], srg * q_rg, 0);
      }
    }
    if constexpr (KQ) {
      S.k = __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(rd, d_off, srg * d_rg, 0));
      S.e = __builtin_bit_cast(u2v, __builtin_amdgcn_raw_buffer_load_b64(re, e_off, srg * e_rg, 0));
    } else {
      S.d = __builtin_amdgcn_raw_buffer_load_b32(rd, d_off, srg * d_rg, 0);
    }
  };
  auto stage_compute = [&](int slot, int buf, int step) {
    const Dx16Slot<FMT>& S = sl[slot];
    {  // dy 2^e -> f16 hi / lo: A fragment tile tl >> 4, lane (tl & 15) + 16 (q4 >> 1), half q4 & 1
      const int nst = n0 + 32 * min(step, max(nsteps - 1, 0));
      f4 dv = dy4[slot];
      if (nst + 32 > a.N) {  // ragged tail of N: columns >= N hold the next token's values
#pragma unroll
        for (int c = 0; c < 4; c++)
          if (nst + 4 * q4 + c >= a.N) dv[c] = 0.0f;
      }
      const half2v h01 = pk_rtz(dv[0] * dsc, dv[1] * dsc), h23 = pk_rtz(dv[2] * dsc, dv[3] * dsc);
      const half2v l01 = pk_rtz(fmaf(dv[0], dsc, -(float)h01.x), fmaf(dv[1], dsc, -(float)h01.y));
      const half2v l23 = pk_rtz(fmaf(dv[2], dsc, -(float)h23.x), fmaf(dv[3], dsc, -(float)h23.y));
      const u2v hv = {__builtin_bit_cast(uint32_t, h01), __builtin_bit_cast(uint32_t, h23)};
      const u2v lv = {__builtin_bit_cast(uint32_t, l01), __builtin_bit_cast(uint32_t, l23)};
      const int fl = (tl & 15) + 16 * (q4 >> 1);
      reinterpret_cast<u2v*>(&sA[buf][tl >> 4][0][fl])[q4 & 1] = hv;
      reinterpret_cast<u2v*>(&sA[buf][tl >> 4][1][fl])[q4 & 1] = lv;
    }
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {  // W: rows li0, li0+1, half hh -> f16 hi / lo (as dx_tile)
      uint32_t hw[4], lw[4];
      if constexpr (KQ) {
        float v[2][4];
#pragma unroll
        for (int r = 0; r < 2; r++) {
          float d, m;
          dq_params<FMT>(0u, comp(S.k, 2 * r + (jb >> 1)), r ? S.e.y : S.e.x, jb, hh, d, m);
          d *= a.wsc;
          m *= a.wsc;
          const uint32_t uu = B8 ? S.q[r][hh] ^ 0x80808080u : (hh ? (S.q[r][0] >> 4) : S.q[r][0]) & 0x0f0f0f0fu;
#pragma unroll
          for (int e = 0; e < 4; e++) v[r][e] = fmaf((float)((uu >> (8 * e)) & 0xffu), d, m);
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const half2v h = pk_rtz(v[0][e], v[1][e]);
          hw[e] = __builtin_bit_cast(uint32_t, h);
          lw[e] = __builtin_bit_cast(uint32_t, pk_rtz(fmaf((float)h.x, neg1, v[0][e]), fmaf((float)h.y, neg1, v[1][e])));
        }
      } else {
        const uint32_t u0 = B8 ? S.q[0][hh] ^ 0x80808080u : (hh ? (S.q[0][0] >> 4) : S.q[0][0]) & 0x0f0f0f0fu;
        const uint32_t u1 = B8 ? S.q[1][hh] ^ 0x80808080u : (hh ? (S.q[1][0] >> 4) : S.q[1][0]) & 0x0f0f0f0fu;
        const uint32_t i01 = __builtin_amdgcn_perm(u1, u0, 0x05010400u), i23 = __builtin_amdgcn_perm(u1, u0, 0x07030602u);
        half2v dp = __builtin_bit_cast(half2v, S.d);
        dp = dp * half2v{(_Float16)a.wsc, (_Float16)a.wsc};
        constexpr _Float16 OFF = B8 ? (_Float16)1152.0f : (_Float16)1032.0f;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const uint32_t src = e < 2 ? i01 : i23;
          const half2v c = sub_h2((e & 1) ? bytes23_to_h2(src) : bytes01_to_h2(src), OFF);
          const half2v h = dp * c;
          const half2v l = __builtin_elementwise_fma(dp, c, -h);
          hw[e] = __builtin_bit_cast(uint32_t, h);
          lw[e] = __builtin_bit_cast(uint32_t, l);
        }
      }
      const int kb = 32 * jb + 16 * hh + 4 * wgg;
      const int nsw = nloc ^ (8 * jb);
#pragma unroll
      for (int e = 0; e < 4; e++) {
        *reinterpret_cast<uint32_t*>(&sW[buf][0][kb + e][nsw]) = hw[e];
        *reinterpret_cast<uint32_t*>(&sW[buf][1][kb + e][nsw]) = lw[e];
      }
    }
    __syncthreads();
    half8 ah[2], al[2];
#pragma unroll
    for (int ts = 0; ts < 2; ts++) {
      ah[ts] = __builtin_bit_cast(half8, sA[buf][ts][0][lane]);
      al[ts] = __builtin_bit_cast(half8, sA[buf][ts][1][lane]);
    }
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
      const int kl = w * 32 + ks * 16 + li;  // column kl lies in block w: rows swizzled by 8 w
      const half8 bh = *reinterpret_cast<const half8*>(&sW[buf][0][kl][8 * (g ^ w)]);
      const half8 bl = *reinterpret_cast<const half8*>(&sW[buf][1][kl][8 * (g ^ w)]);
#pragma unroll
      for (int ts = 0; ts < 2; ts++) {
        acc[ts][ks] = mfma_f16(ah[ts], bh, acc[ts][ks]);
        acc[ts][ks] = mfma_f16(al[ts], bh, acc[ts][ks]);
        acc[ts][ks] = mfma_f16(ah[ts], bl, acc[ts][ks]);
      }
    }
  };
#pragma unroll
  for (int s0 = 0; s0 < D - 1; s0++) issue(s0, s0);
  for (int st0 = 0; st0 < nsteps; st0 += D) {
#pragma unroll
    for (int s0 = 0; s0 < D; s0++) {
      issue((s0 + D - 1) % D, st0 + s0 + D - 1);
      __builtin_amdgcn_sched_barrier(0);
      if (st0 + s0 < nsteps) stage_compute(s0, (st0 + s0) & 1, st0 + s0);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // rows back to dy's scale (and W's), then the partial in the 64-token fragment order: this
  // workgroup's wave w is wave 4 wt + w of the 64-token tile t0 / 64 (wt = (t0 % 64) / 32)
#pragma unroll
  for (int ts = 0; ts < 2; ts++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float sv = sInv[16 * ts + 4 * g + i];
#pragma unroll
      for (int ks = 0; ks < 2; ks++) acc[ts][ks][i] *= sv;
    }
  const int wt = (t0 >> 5) & 1;
  f4* out = reinterpret_cast<f4*>(a.part) + ((((int64_t)sp * ntt + (t0 >> 6)) * Kc + kc) * 8 + 4 * wt + w) * 256 + lane;
#pragma unroll
  for (int ts = 0; ts < 2; ts++)
#pragma unroll
    for (int ks = 0; ks < 2; ks++) out[(ts * 2 + ks) * 64] = acc[ts][ks];
}

extern "C" __global__ __launch_bounds__(256) void rtq_dx32_q4_0(DxArgs a) { dx32_tile<FMT_Q4_0>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_dx32_q8_0(DxArgs a) { dx32_tile<FMT_Q8_0>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_dx32_q4_k(DxArgs a) { dx32_tile<FMT_Q4_K>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_dx32_q6_k(DxArgs a) { dx32_tile<FMT_Q6_K>(a); }

extern "C" __global__ __launch_bounds__(256) void rtq_dxv1_q4_0(DxArgs a) { dxv1_tile<FMT_Q4_0>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_dxv1_q8_0(DxArgs a) { dxv1_tile<FMT_Q8_0>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_dxv1_q4_k(DxArgs a) { dxv1_tile<FMT_Q4_K>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_dxv1_q6_k(DxArgs a) { dxv1_tile<FMT_Q6_K>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_dx16_q4_0(DxArgs a) { dx16_tile<FMT_Q4_0>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_dx16_q8_0(DxArgs a) { dx16_tile<FMT_Q8_0>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_dx16_q4_k(DxArgs a) { dx16_tile<FMT_Q4_K>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_dx16_q6_k(DxArgs a) { dx16_tile<FMT_Q6_K>(a); }

// two 64-token workgroups per CU (four waves per SIMD: at most 128 VGPRs)
extern "C" __global__ __launch_bounds__(512, 4) void rtq_dx_q4_0(DxArgs a) { dx_tile<FMT_Q4_0, 64>(a); }
extern "C" __global__ __launch_bounds__(512, 4) void rtq_dx_q8_0(DxArgs a) { dx_tile<FMT_Q8_0, 64>(a); }
extern "C" __global__ __launch_bounds__(512, 4) void rtq_dx_q4_k(DxArgs a) { dx_tile<FMT_Q4_K, 64>(a); }
extern "C" __global__ __launch_bounds__(512, 4) void rtq_dx_q6_k(DxArgs a) { dx_tile<FMT_Q6_K, 64>(a); }
extern "C" __global__ __launch_bounds__(512) void rtq_dxw_q4_0(DxArgs a) { dx_tile<FMT_Q4_0, 256>(a); }
extern "C" __global__ __launch_bounds__(512) void rtq_dxw_q8_0(DxArgs a) { dx_tile<FMT_Q8_0, 256>(a); }
extern "C" __global__ __launch_bounds__(512) void rtq_dxw_q4_k(DxArgs a) { dx_tile<FMT_Q4_K, 256>(a); }
extern "C" __global__ __launch_bounds__(512) void rtq_dxw_q6_k(DxArgs a) { dx_tile<FMT_Q6_K, 256>(a); }

// ============================================================== backward finish
// dx[t][k] = [dx[t][k] +] sum over splits s (in order) of the partials [+ sum_j g[t][j] A[j][k]]
//   (FrozenMatmul::backward_input accumulates, src/frozen.rs:19-20; Linear::backward returns
//    w.backward_input(dy) + g.A, src/linear.rs:100-101,115-118)
// gb[n][j] += sum_t (s*dy[t][n]) h[t][j]   (matmul_tn_acc, src/linear.rs:109)
// ga[j][k] += sum_t g[t][j] x[t][k]        (matmul_tn_acc, src/linear.rs:113)
// gb / ga: one R x 16 tile (R = 16 E rows m of X = s.dy or x, 16 ranks j) per workgroup: E = 4, or
// E = 1 where 64-row tiles would leave most CUs without a workgroup.  The NW waves split the tokens
// and contract 4 tokens per step with E f32 MFMAs (MFMA e takes rows m0 + E rho + e, rho the MFMA's
// row, so a lane's E values of a token row are one load); their tiles are added in LDS in wave order
// (single writer, fixed order).  The accumulated outputs are read at the start, so that load's
// latency overlaps the contraction.  GB: tile b of gb (X = dy, H = h), otherwise of ga (X = x, H = g).
template <int E>
struct FloatVec;
template <>
struct FloatVec<1> {
  using T = float;
};
template <>
struct FloatVec<4> {
  using T = f4;
};
template <int NW, int E, bool GB>
__device__ __forceinline__ void lora_grad_tile(const LoraGradArgs& a, int b, float* red) {
  constexpr int LDR = 17;  // LDS row stride of a wave's R x 16 tile (the four lane groups on different banks)
  constexpr int R = 16 * E, NO = (R * 16 + NW * 64 - 1) / (NW * 64);  // outputs per thread
  using V = typename FloatVec<E>::T;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, li = lane & 15, g = lane >> 4;
  const int jt = (a.r + 15) / 16, m0 = (b / jt) * R, j0 = (b % jt) * 16;
  const int M = GB ? a.N : a.K;
  // block-diagonal adapter: only tiles that meet a member's block (uniform exit)
  if (GB && !rb_any(a.rb, m0, min(m0 + R, a.N), j0, min(j0 + 16, a.r))) return;
  // output o of this thread: gb: consecutive threads take consecutive ranks of a row; ga: consecutive
  // columns of a rank
  auto out_at = [&](int o, int& m, int& j) {
    m = m0 + (GB ? o >> 4 : o % R);
    j = j0 + (GB ? o & 15 : o / R);
  };
  float prev[NO];
#pragma unroll
  for (int q = 0; q < NO; q++) {
    const int o = threadIdx.x + q * NW * 64;
    int m, j;
    out_at(o, m, j);
    prev[q] = 0.0f;
    if (o < R * 16 && m < M && j < a.r) prev[q] = GB ? a.gb[(int64_t)m * a.r + j] : a.ga[(int64_t)j * a.K + m];
  }
  const float* X = GB ? a.dy : a.x;  // [T x M]
  const float* H = GB ? a.h : a.g;   // [T x r]
  const int tper = (a.T + NW * 16 - 1) / (NW * 16) * 16;  // tokens per wave, multiple of 16
  const int tb = w * tper, te = min(tb + tper, a.T);
  const int mc = m0 + E * li, jc = j0 + li;
  const bool vec = (M % E) == 0;  // E-aligned rows (always for x: K % 32 == 0)
  f4 acc[E];
#pragma unroll
  for (int e = 0; e < E; e++) acc[e] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  for (int t32 = tb; t32 < te; t32 += 32) {  // 32 tokens: all loads, then up to 8 E MFMAs
    const int nv = min(2, (te - t32 + 15) / 16);  // 16-token groups with tokens (wave-uniform)
    V xv[2][4];
    float hv[2][4];
#pragma unroll
    for (int v = 0; v < 2; v++)
      if (v < nv)
#pragma unroll
        for (int u = 0; u < 4; u++) {
          const int t = t32 + 16 * v + 4 * u + g, tc = min(t, a.T - 1);
          const bool tin = t < te;
          const float* xr = X + (int64_t)tc * M;
          if (vec) {
            const V x4 = *reinterpret_cast<const V*>(xr + min(mc, M - E));
            xv[v][u] = (tin && mc < M) ? x4 : V{};
          } else {
            float* xe = reinterpret_cast<float*>(&xv[v][u]);
#pragma unroll
            for (int e = 0; e < E; e++) xe[e] = (tin && mc + e < M) ? xr[min(mc + e, M - 1)] : 0.0f;
          }
          const float hh = H[(int64_t)tc * a.r + min(jc, a.r - 1)];
          hv[v][u] = (tin && jc < a.r) ? hh : 0.0f;
        }
#pragma unroll
    for (int v = 0; v < 2; v++)
      if (v < nv)
#pragma unroll
        for (int u = 0; u < 4; u++) {
          const float* xe = reinterpret_cast<const float*>(&xv[v][u]);
#pragma unroll
          for (int e = 0; e < E; e++)  // s.dy (src/linear.rs:108) for gb; x for ga
            acc[e] = mfma_f32(GB ? __fmul_rn(xe[e], a.s) : xe[e], hv[v][u], acc[e]);
        }
  }
  // lane (rank li, group g): element i of acc[e] is row m0 + E (4g + i) + e
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int e = 0; e < E; e++) red[w * R * LDR + (E * (4 * g + i) + e) * LDR + li] = acc[e][i];
  __syncthreads();
#pragma unroll
  for (int q = 0; q < NO; q++) {
    const int o = threadIdx.x + q * NW * 64;
    if (o >= R * 16) break;
    const int mr = GB ? o >> 4 : o % R, jr = GB ? o & 15 : o / R;
    float sum = 0.0f;
#pragma unroll
    for (int ww = 0; ww < NW; ww++) sum += red[ww * R * LDR + mr * LDR + jr];
    int m, j;
    out_at(o, m, j);
    if (m < M && j < a.r) {
      if (GB) {
        if (rb_keep(a.rb, m, j)) a.gb[(int64_t)m * a.r + j] = prev[q] + sum;
      } else {
        a.ga[(int64_t)j * a.K + m] = prev[q] + sum;
      }
    }
  }
}

// One grid, three kinds of workgroups: gb tiles, ga tiles (lora_grad_tile), then dx: one wave per
// 16 x 16 quarter of a dx-kernel fragment (the dx kernel's partial layout) or per token and 64
// columns (row-major partials).  NW = 4, or 16 for long token ranges.  DXO: dx workgroups alone
// (n_gb = n_ga = 0: dA / dB deferred or no adapter) over at most four splits, loading four
// partials at a time (the same split order; a quarter of the load registers).
// dx[t, k0 .. k0+3] from its summed partials: + g[t] . A[:, k0 .. k0+3] (src/linear.rs:115-118),
// then stored / accumulated, or (sw) taken as SwiGLU's dh (accumulate is off there)
__device__ __forceinline__ void finish_row4(const LoraGradArgs& a, int t, int k0, f4 sum, bool sw) {
  if (a.g) {
    f4 ga = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int j = 0; j < a.r; j++) {
      const float gv = a.g[(int64_t)t * a.r + j];
      const float* av = a.la + (int64_t)j * a.K + k0;  // caller's A: no alignment assumed
#pragma unroll
      for (int e = 0; e < 4; e++) ga[e] = fmaf(gv, av[e], ga[e]);
    }
    sum += ga;
  }
  if (sw) {
    const int64_t o = (int64_t)t * a.swld + k0;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const float gv = a.swg[o + e], uv = a.swu[o + e];
      a.swdg[o + e] = (sum[e] * uv) * rtq_silu_grad(gv);
      a.swdu[o + e] = sum[e] * rtq_silu(gv);
      if (a.sw_keep) a.dx[(int64_t)t * a.K + k0 + e] = sum[e];
    }
  } else {
    float* p = a.dx + (int64_t)t * a.K + k0;
#pragma unroll
    for (int e = 0; e < 4; e++) p[e] = a.accumulate ? p[e] + sum[e] : sum[e];
  }
}

template <int NW, int E, bool DXO = false>
__device__ __forceinline__ void bwd_finish(const LoraGradArgs& a) {
  __shared__ float red[DXO ? 1 : NW * 16 * E * 17];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, li = lane & 15, g = lane >> 4;
  const int b = blockIdx.x;
  if (!DXO && b < a.n_gb) {
    lora_grad_tile<NW, E, true>(a, b, red);
  } else if (!DXO && b < a.n_gb + a.n_ga) {
    lora_grad_tile<NW, E, false>(a, b - a.n_gb, red);
  } else if (a.part_rows) {
    // dx from row-major partials: wave per (token t, 64 columns); lane (k4 = li, split subset g)
    // sums splits g, g+4, ... of four columns, the subsets are combined by shuffles (fixed order)
    const int nseg = (a.K + 63) / 64;
    const int f = (b - a.n_gb - a.n_ga) * NW + w;
    if (f >= a.T * nseg) return;  // whole wave exits together; no barriers in this branch
    const int t = f / nseg, k0 = (f % nseg) * 64 + 4 * li;
    const bool kin = k0 < a.K;  // K % 32 == 0: four columns in or out together
    f4 sum = {0.0f, 0.0f, 0.0f, 0.0f};
    const f4* pp = reinterpret_cast<const f4*>(a.part + (int64_t)t * a.K + min(k0, a.K - 4));
    const int64_t sstride = (int64_t)a.T * a.K / 4;  // f4 per split
    constexpr int PRL = DXO ? 1 : 16;  // loads in flight per lane, summed in order
    for (int s0 = g; s0 < a.nsplit; s0 += 4 * PRL) {
      f4 v[PRL];
#pragma unroll
      for (int q = 0; q < PRL; q++) v[q] = pp[(int64_t)min(s0 + 4 * q, a.nsplit - 1) * sstride];
#pragma unroll
      for (int q = 0; q < PRL; q++)
        if (s0 + 4 * q < a.nsplit) sum += v[q];
    }
#pragma unroll
    for (int e = 0; e < 4; e++) {
      sum[e] += __shfl_xor(sum[e], 16);
      sum[e] += __shfl_xor(sum[e], 32);
    }
    if (g == 0 && kin) finish_row4(a, t, k0, sum, NW == 4 && a.swg);
  } else {
    // dx quarter fq = (b - n_gb - n_ga) * NW + w: fragment f = fq / 4 of the dx kernel's partials
    // (tile f / 8 = token tile * Kc + K chunk, its wave f % 8 = (wt, wk)), quarter q = fq % 4 =
    // (ts, ks); lane element i <-> row t0 + 32wt + 16ts + 4g + i, column 128kc + 32wk + 16ks + li
    // (the MFMA output layout of both kernels).  All splits' loads are issued at once.
    const int Kc = (a.K + 127) / 128, ntt = (a.T + 63) / 64;
    const int fq = (b - a.n_gb - a.n_ga) * NW + w;
    if (fq >= ntt * Kc * 8 * 4) return;  // whole wave exits together; no barriers in this branch
    const int f = fq >> 2, q = fq & 3, ts = q >> 1, ks = q & 1;
    const int tile = f >> 3, dw = f & 7, wt = dw >> 2, wk = dw & 3;
    const int t0 = (tile / Kc) * 64 + wt * 32 + ts * 16, k0 = (tile % Kc) * 128 + wk * 32 + ks * 16;
    const f4* pp = reinterpret_cast<const f4*>(a.part) + (int64_t)f * 256 + q * 64 + lane;
    const int64_t sstride = (int64_t)ntt * Kc * 8 * 256;  // f4 per split
    const int trow = t0 + li, kcol = k0 + li;
    // g . A operands (f32 MFMA; lane: token 4g + i, column li) of rank chunk jj; the first MAXJ
    // chunks' loads are issued with the partials', so the tile waits for one round of loads
    auto ga_ops = [&](int jj, float* gv, float* av) {
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int j = 16 * jj + 4 * u + g, jc = min(j, a.r - 1);
        const float x = a.g[(int64_t)min(trow, a.T - 1) * a.r + jc];
        const float y = a.la[(int64_t)jc * a.K + min(kcol, a.K - 1)];
        gv[u] = (trow < a.T && j < a.r) ? x : 0.0f;
        av[u] = (kcol < a.K && j < a.r) ? y : 0.0f;
      }
    };
    constexpr int MAXJ = NW == 16 ? 2 : 4;  // (sixteen-wave workgroups hold 128 VGPRs per lane)
    const int nj = a.g ? (a.r + 15) / 16 : 0;
    float gv[MAXJ][4], av[MAXJ][4];
#pragma unroll
    for (int jj = 0; jj < MAXJ; jj++)
      if (jj < nj) ga_ops(jj, gv[jj], av[jj]);
    // SwiGLU's g, u of these outputs (accumulate off, 4-wave finish only), loaded with the partials
    const bool sw = NW == 4 && a.swg;  // uniform
    float swgv[4], swuv[4];
    if (sw) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int64_t o = (int64_t)min(t0 + 4 * g + i, a.T - 1) * a.swld + min(kcol, a.K - 1);
        swgv[i] = a.swg[o];
        swuv[i] = a.swu[o];
      }
    }
    constexpr int MAXS = DXO ? 4 : NW == 16 ? 8 : 16;  // partials loaded at once; more splits are summed MAXS at a time
    f4 ps = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int c0 = 0; c0 < a.nsplit; c0 += MAXS) {
      f4 v[MAXS];
#pragma unroll
      for (int sp = 0; sp < MAXS; sp++)
        if (c0 + sp < a.nsplit) v[sp] = pp[(int64_t)(c0 + sp) * sstride];
      if (c0 == 0) ps = v[0];
#pragma unroll
      for (int sp = 0; sp < MAXS; sp++)
        if ((c0 > 0 || sp > 0) && c0 + sp < a.nsplit) ps += v[sp];  // split order
    }
    f4 ga = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int jj = 0; jj < MAXJ; jj++)
      if (jj < nj)
#pragma unroll
        for (int u = 0; u < 4; u++) ga = mfma_f32(gv[jj][u], av[jj][u], ga);
    for (int jj = MAXJ; jj < nj; jj++) {
      float gq[4], aq[4];
      ga_ops(jj, gq, aq);
#pragma unroll
      for (int u = 0; u < 4; u++) ga = mfma_f32(gq[u], aq[u], ga);
    }
    if (kcol < a.K) {
      if (sw) {  // SwiGLU backward of dh = the sum
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int t = t0 + 4 * g + i;
          if (t < a.T) {
            const float dh = a.g ? ps[i] + ga[i] : ps[i];
            const int64_t o = (int64_t)t * a.swld + kcol;
            a.swdg[o] = (dh * swuv[i]) * rtq_silu_grad(swgv[i]);
            a.swdu[o] = dh * rtq_silu(swgv[i]);
            if (a.sw_keep) a.dx[(int64_t)t * a.K + kcol] = dh;
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int t = t0 + 4 * g + i;
          if (t < a.T) {
            float* p = &a.dx[(int64_t)t * a.K + kcol];
            float o = a.accumulate ? *p + ps[i] : ps[i];
            if (a.g) o += ga[i];
            *p = o;
          }
        }
      }
    }
  }
}

// the dA / dB tiles of several linears (a decoder block's, deferred to one launch so that their
// load -> contract -> reduce chains overlap instead of running one launch after another)
template <int NW>
__device__ __forceinline__ void lora_grads(const LoraGradBatch& B) {
  __shared__ float red[NW * 64 * 17];
  const int b = blockIdx.x;
  int j = 0;
  while (j + 1 < B.njobs && b >= B.start[j + 1]) j++;  // uniform over the workgroup
  const LoraGradArgs& a = B.job[j];
  const int lb = b - B.start[j];
  if (lb < a.n_gb)
    lora_grad_tile<NW, 4, true>(a, lb, red);
  else if (lb < a.n_gb + a.n_ga)
    lora_grad_tile<NW, 4, false>(a, lb - a.n_gb, red);
}

extern "C" __global__ __launch_bounds__(256) void rtq_lora_grads(LoraGradBatch b) { lora_grads<4>(b); }
extern "C" __global__ __launch_bounds__(1024) void rtq_lora_grads16(LoraGradBatch b) { lora_grads<16>(b); }

// the same over a device job table (a whole step's adapted linears in one launch)
template <int NW>
__device__ __forceinline__ void lora_grads_t(const LoraGradTable& T) {
  __shared__ float red[NW * 64 * 17];
  const int b = blockIdx.x;
  const int j = __builtin_amdgcn_readfirstlane(T.map[2 * b]), lb = __builtin_amdgcn_readfirstlane(T.map[2 * b + 1]);
  const LoraGradArgs a = T.job[j];
  if (lb < a.n_gb)
    lora_grad_tile<NW, 4, true>(a, lb, red);
  else if (lb < a.n_gb + a.n_ga)
    lora_grad_tile<NW, 4, false>(a, lb - a.n_gb, red);
}
extern "C" __global__ __launch_bounds__(256) void rtq_lora_grads_t(LoraGradTable t) { lora_grads_t<4>(t); }
extern "C" __global__ __launch_bounds__(1024) void rtq_lora_grads_t16(LoraGradTable t) { lora_grads_t<16>(t); }
extern "C" __global__ __launch_bounds__(256) void rtq_bwd_finish(LoraGradArgs a) { bwd_finish<4, 4>(a); }
extern "C" __global__ __launch_bounds__(1024) void rtq_bwd_finish16(LoraGradArgs a) { bwd_finish<16, 4>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_bwd_finish_dx(LoraGradArgs a) { bwd_finish<4, 4, true>(a); }

// dx from row-major partials of many splits (rtq_dx16_* / rtq_dxv1_* over a long weight; no dA / dB
// tiles): a workgroup per (token t, 64 columns), four times the workgroups of the wave-per-segment
// form.  Wave w, lane (k4 = li, g) sums splits 4w + g, 4w + g + 16, ... in order (eight loads in
// flight); the sixteen subsets are combined by shuffles (g), then through LDS (w = 0, 1, 2, 3)
extern "C" __global__ __launch_bounds__(256) void rtq_bwd_finish_rows(LoraGradArgs a) {
  __shared__ f4 red[3][16];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, li = lane & 15, g = lane >> 4;
  const int nseg = (a.K + 63) / 64;
  if ((int)blockIdx.x >= a.T * nseg) return;  // whole workgroup exits together, before the barrier
  const int t = blockIdx.x / nseg, k0 = (blockIdx.x % nseg) * 64 + 4 * li;
  const bool kin = k0 < a.K;  // K % 32 == 0: four columns in or out together
  const f4* pp = reinterpret_cast<const f4*>(a.part + (int64_t)t * a.K + min(k0, a.K - 4));
  const int64_t sstride = (int64_t)a.T * a.K / 4;  // f4 per split
  constexpr int PRL = 8;
  f4 sum = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int s0 = 4 * w + g; s0 < a.nsplit; s0 += 16 * PRL) {
    f4 v[PRL];
#pragma unroll
    for (int q = 0; q < PRL; q++) v[q] = pp[(int64_t)min(s0 + 16 * q, a.nsplit - 1) * sstride];
#pragma unroll
    for (int q = 0; q < PRL; q++)
      if (s0 + 16 * q < a.nsplit) sum += v[q];
  }
#pragma unroll
  for (int e = 0; e < 4; e++) {
    sum[e] += __shfl_xor(sum[e], 16);
    sum[e] += __shfl_xor(sum[e], 32);
  }
  if (w > 0 && g == 0) red[w - 1][li] = sum;
  __syncthreads();
  if (w == 0 && g == 0 && kin) {
    sum += red[0][li];
    sum += red[1][li];
    sum += red[2][li];
    finish_row4(a, t, k0, sum, a.swg != nullptr);
  }
}


// ============================================================== trainer-native weights
// rows [r0, r0 + count) of an F32 (copy) or TQ8_0 weight (0 + d * q: q8_axpy(1) into zeros,
// src/frozen.rs:172-176, bit-exact) into out [count][K]; the same kernel dequantises a whole TQ8_0
// weight for the f32 GEMMs
extern "C" __global__ __launch_bounds__(256) void rtq_dense_rows(DenseArgs a) {
  const int64_t n = a.count * a.K;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t k = i % a.K;
    int64_t r = a.r0 + i / a.K;
    if (a.idx) {
      r = a.idx[i / a.K];
      if (r < 0 || r >= a.N) {  // out-of-range id: NaN row, nothing read
        a.out[i] = __builtin_nanf("");
        continue;
      }
    }
    if (a.w)
      a.out[i] = a.w[r * a.K + k];
    else
      a.out[i] = 0.0f + a.sc[r * (a.K / 32) + k / 32] * (float)a.qs[r * a.K + k];
  }
}

// y[t][n] += bias[n] (src/linear.rs:77-83), t < count
extern "C" __global__ __launch_bounds__(256) void rtq_dense_bias(DenseArgs a) {
  const int64_t n = a.count * a.N;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    a.out[i] = a.out[i] + a.bias[i % a.N];
}

// ============================================================== row dequant (FrozenMatmul::row)
// embedding gather: weight row of out row rl; an id outside [0, rows) gives a NaN block, nothing read
__device__ __forceinline__ bool gather_row(const RowArgs& a, int rl, int b, int* n) {
  const int r = a.idx[rl];
  if (r >= 0 && r < a.rows) {
    *n = r;
    return true;
  }
  float* out = a.out + (int64_t)rl * a.K + b * 32;
#pragma unroll
  for (int e = 0; e < 32; e++) out[e] = __builtin_nanf("");
  return false;
}

// One thread per (row, 32-element block); bit-exact ggml dequant: (q - 8) * d, q * d.
extern "C" __global__ __launch_bounds__(256) void rtq_rows_q4_0(RowArgs a) {
  const int nb = a.K / 32, Kc = a.Kp / 128;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)a.count * nb) return;
  const int rl = (int)(idx / nb), b = (int)(idx % nb);
  int n = a.r0 + rl;
  if (a.idx && !gather_row(a, rl, b, &n)) return;
  const int rg = n >> 4, li = n & 15, kc = b >> 2, j = b & 3;
  const u4v* q = reinterpret_cast<const u4v*>(a.wq) + (int64_t)(rg * Kc + kc) * 64;
  const float d = h2f(a.wd[RTQ_WD_INDEX(rg, kc, Kc, li, j)]);
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
  int n = a.r0 + rl;
  if (a.idx && !gather_row(a, rl, b, &n)) return;
  const int rg = n >> 4, li = n & 15, kc = b >> 2, j = b & 3;
  const u4v* q = reinterpret_cast<const u4v*>(a.wq) + (int64_t)(rg * Kc + kc) * 128 + (j >> 1) * 64;
  const float d = h2f(a.wd[RTQ_WD_INDEX(rg, kc, Kc, li, j)]);
  float* out = a.out + (int64_t)rl * a.K + b * 32;
#pragma unroll
  for (int gg = 0; gg < 4; gg++) {
    const u4v v = q[li + 16 * gg];
    const uint32_t lo = (j & 1) ? v.z : v.x, hi = (j & 1) ? v.w : v.y;
#pragma unroll
    for (int s = 0; s < 4; s++) {
      out[4 * gg + s] = (float)(int8_t)((lo >> (8 * s)) & 0xff) * d;
      out[16 + 4 * gg + s] = (float)(int8_t)((hi >> (8 * s)) & 0xff) * d;
    }
  }
}

// K-quants, one thread per (row, 32-element block), bit-exact with ggml's dequantisation:
//   Q4_K: (d*sc)*u - dmin*m (two roundings at most: the products are exact);
//   Q6_K: (d*sc)*q, sc of each 16-element half (exact product, then one rounding).
template <int FMT>
__device__ __forceinline__ void rows_kquant(const RowArgs& a) {
  const int nb = a.K / 32, Kc = a.Kp / 128;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)a.count * nb) return;
  const int rl = (int)(idx / nb), b = (int)(idx % nb);
  int n = a.r0 + rl;
  if (a.idx && !gather_row(a, rl, b, &n)) return;
  const int rg = n >> 4, li = n & 15, kc = b >> 2, j = b & 3;
  const uint32_t kw = a.wd[RTQ_WR_INDEX(rg, kc, Kc, li, j)];
  const uint32_t ev = a.wsb[RTQ_WSB_INDEX(rg, kc >> 1, Kc >> 1, li)];
  const float dsb = h2f((uint16_t)(ev & 0xffffu));
  float* out = a.out + (int64_t)rl * a.K + b * 32;
  if (FMT == FMT_Q4_K) {
    const float sc = __fmul_rn(dsb, (float)(kw & 0x3fu));
    const float mn = __fmul_rn(h2f((uint16_t)(ev >> 16)), (float)((kw >> 8) & 0x3fu));
    const u4v* q = reinterpret_cast<const u4v*>(a.wq) + (int64_t)(rg * Kc + kc) * 64;
#pragma unroll
    for (int gg = 0; gg < 4; gg++) {
      const uint32_t w = comp(q[li + 16 * gg], j);
#pragma unroll
      for (int s = 0; s < 4; s++) {
        const uint32_t byte = (w >> (8 * s)) & 0xffu;
        out[4 * gg + s] = __fsub_rn(__fmul_rn(sc, (float)(byte & 0xfu)), mn);
        out[16 + 4 * gg + s] = __fsub_rn(__fmul_rn(sc, (float)(byte >> 4)), mn);
      }
    }
  } else {
    const float s0 = __fmul_rn(dsb, (float)(int)(int8_t)(kw & 0xffu));
    const float s1 = __fmul_rn(dsb, (float)(int)(int8_t)((kw >> 8) & 0xffu));
    const u4v* q = reinterpret_cast<const u4v*>(a.wq) + (int64_t)(rg * Kc + kc) * 128 + (j >> 1) * 64;
#pragma unroll
    for (int gg = 0; gg < 4; gg++) {
      const u4v v = q[li + 16 * gg];
      const uint32_t lo = (j & 1) ? v.z : v.x, hi = (j & 1) ? v.w : v.y;
#pragma unroll
      for (int s = 0; s < 4; s++) {
        out[4 * gg + s] = __fmul_rn(s0, (float)(int8_t)((lo >> (8 * s)) & 0xffu));
        out[16 + 4 * gg + s] = __fmul_rn(s1, (float)(int8_t)((hi >> (8 * s)) & 0xffu));
      }
    }
  }
}

extern "C" __global__ __launch_bounds__(256) void rtq_rows_q4_k(RowArgs a) { rows_kquant<FMT_Q4_K>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_rows_q6_k(RowArgs a) { rows_kquant<FMT_Q6_K>(a); }

// ============================================================== LM head + cross-entropy
// Model::head (src/model.rs:561-609) for all targets at once: rtq_head_norm (gather + RMSNorm),
// the lm_head forward (the kernels above), rtq_head_max / _sum / _grad over G vocabulary slices per
// row (softmax_row, src/ops.rs:238-247: p = exp(v - max) in f32, normaliser summed in f64, the
// gradient w (p / s - onehot) written over the logits), the lm_head backward_input, and
// rtq_head_norm_bwd (rmsnorm_backward, src/ops.rs:39-56, added into dx at the target positions).
// A target outside [0, t) x [0, V) reads nothing: its normalised row is 0, logp NaN, gradient 0.

__device__ __forceinline__ bool head_target_ok(const HeadArgs& a, int i) {
  const int p = a.pos[i], k = a.tok[i];
  return p >= 0 && p < a.t && k >= 0 && k < a.V;
}

// sum over the 256 threads of a workgroup; every thread gets the same value
template <class T>
__device__ __forceinline__ T block_sum256(T v, T* red) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
  __syncthreads();  // red may still be read from a previous call
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

__device__ __forceinline__ float block_max256(float v, float* red) {
  v = wave_max(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// calls f(j, logit) for every element j of slice g of row i (float4 loads when rows are 16 B aligned)
template <class F>
__device__ __forceinline__ void head_slice(const HeadArgs& a, const float* row, int j0, int j1, F&& f) {
  if ((a.V & 3) == 0) {
    const f4* r4 = reinterpret_cast<const f4*>(row);
    for (int q = j0 / 4 + (int)threadIdx.x; q < j1 / 4; q += 256) {
      const f4 v = r4[q];
      f(4 * q, v[0]);
      f(4 * q + 1, v[1]);
      f(4 * q + 2, v[2]);
      f(4 * q + 3, v[3]);
    }
  } else {
    for (int j = j0 + (int)threadIdx.x; j < j1; j += 256) f(j, row[j]);
  }
}

// grid n: ns[i] = (x[pos[i]] * ir) * (norm + off), ir = 1 / sqrt(dot(x, x) / d + eps)
extern "C" __global__ __launch_bounds__(256) void rtq_head_norm(HeadArgs a) {
  __shared__ float red[4];
  const int i = blockIdx.x;
  float* out = a.ns + (int64_t)i * a.d;
  if (!head_target_ok(a, i)) {
    for (int k = threadIdx.x; k < a.d; k += 256) out[k] = 0.0f;
    if (threadIdx.x == 0) a.inv[i] = 0.0f;
    return;
  }
  const float* xr = a.x + (int64_t)a.pos[i] * a.d;
  float s = 0.0f;
  for (int k = threadIdx.x; k < a.d; k += 256) s = s + xr[k] * xr[k];
  s = block_sum256(s, red);
  const float ir = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(s, (float)a.d) + a.eps));
  for (int k = threadIdx.x; k < a.d; k += 256) out[k] = (xr[k] * ir) * (a.norm[k] + a.off);
  if (threadIdx.x == 0) a.inv[i] = ir;
}

// grid (G, n): maximum of slice g of row i
extern "C" __global__ __launch_bounds__(256) void rtq_head_max(HeadArgs a) {
  __shared__ float red[4];
  const int g = blockIdx.x, i = blockIdx.y;
  const float* row = a.logits + (int64_t)i * a.V;
  const int j0 = g * a.L, j1 = min(a.V, j0 + a.L);
  float m = -__builtin_inff();
  head_slice(a, row, j0, j1, [&](int, float v) { m = fmaxf(m, v); });
  m = block_max256(m, red);
  if (threadIdx.x == 0) a.pmax[(int64_t)i * a.G + g] = m;
}

__device__ __forceinline__ float head_row_max(const HeadArgs& a, int i) {
  float m = -__builtin_inff();
  for (int q = 0; q < a.G; q++) m = fmaxf(m, a.pmax[(int64_t)i * a.G + q]);
  return m;
}

// grid (G, n): sum over slice g of row i of exp(v - max), each term rounded to f32, summed in f64
extern "C" __global__ __launch_bounds__(256) void rtq_head_sum(HeadArgs a) {
  __shared__ double red[4];
  const int g = blockIdx.x, i = blockIdx.y;
  const float* row = a.logits + (int64_t)i * a.V;
  const int j0 = g * a.L, j1 = min(a.V, j0 + a.L);
  const float m = head_row_max(a, i);
  double s = 0.0;
  head_slice(a, row, j0, j1, [&](int, float v) { s += (double)expf(v - m); });
  s = block_sum256(s, red);
  if (threadIdx.x == 0) a.psum[(int64_t)i * a.G + g] = s;
}

// grid (G, n): log-prob and hit of target i (by the slice holding its token), then, with weights,
// dlogits = w * (exp(v - max) * (f32)(1 / s)), minus w at the token, over the slice
extern "C" __global__ __launch_bounds__(256) void rtq_head_grad(HeadArgs a) {
  const int g = blockIdx.x, i = blockIdx.y;
  float* row = a.logits + (int64_t)i * a.V;
  const int j0 = g * a.L, j1 = min(a.V, j0 + a.L);
  const float m = head_row_max(a, i);
  double s = 0.0;
  for (int q = 0; q < a.G; q++) s += a.psum[(int64_t)i * a.G + q];
  const float inv = (float)(1.0 / s);
  const float lse = m + (float)log(s);
  const bool ok = head_target_ok(a, i);
  const int tk = ok ? a.tok[i] : -1;
  if (threadIdx.x == 0) {
    if (ok && tk >= j0 && tk < j1) {
      const float tl = row[tk];
      a.logp[i] = tl - lse;
      a.hit[i] = tl >= m ? 1 : 0;
    } else if (!ok && g == 0) {
      a.logp[i] = __builtin_nanf("");
      a.hit[i] = 0;
    }
  }
  if (!a.wts) return;
  __syncthreads();  // the target's logit is read before its slice is overwritten
  const float wi = ok ? a.wts[i] : 0.0f;
  if ((a.V & 3) == 0) {
    f4* r4 = reinterpret_cast<f4*>(row);
    for (int q = j0 / 4 + (int)threadIdx.x; q < j1 / 4; q += 256) {
      f4 v = r4[q];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        float dl = ok ? wi * (expf(v[e] - m) * inv) : 0.0f;
        if (4 * q + e == tk) dl = dl - wi;
        v[e] = dl;
      }
      r4[q] = v;
    }
  } else {
    for (int j = j0 + (int)threadIdx.x; j < j1; j += 256) {
      float dl = ok ? wi * (expf(row[j] - m) * inv) : 0.0f;
      if (j == tk) dl = dl - wi;
      row[j] = dl;
    }
  }
}

// grid n: the first target at each position writes that dx row: 0 + the rmsnorm_backward of every
// target at the position, in target order (dx[pos] += dxs, src/model.rs:600-604)
extern "C" __global__ __launch_bounds__(256) void rtq_head_norm_bwd(HeadArgs a) {
  __shared__ float red[4];
  const int i = blockIdx.x;
  if (!head_target_ok(a, i)) return;
  const int p = a.pos[i];
  int earlier = 0;
  for (int j = threadIdx.x; j < i; j += 256) earlier |= (a.pos[j] == p && head_target_ok(a, j)) ? 1 : 0;
  if (__syncthreads_or(earlier)) return;
  // later targets at the same position (rare): then walk them in order, else only target i
  int later = 0;
  for (int j = i + 1 + (int)threadIdx.x; j < a.n; j += 256) later |= (a.pos[j] == p && head_target_ok(a, j)) ? 1 : 0;
  const int jend = __syncthreads_or(later) ? a.n : i + 1;
  const float* xr = a.x + (int64_t)p * a.d;
  float* o = a.dx + (int64_t)p * a.d;
  for (int j = i; j < jend; j++) {
    if (a.pos[j] != p || !head_target_ok(a, j)) continue;
    const float ir = a.inv[j];
    const float* dr = a.dns + (int64_t)j * a.d;
    float s = 0.0f;
    for (int k = threadIdx.x; k < a.d; k += 256) s = s + (dr[k] * (a.norm[k] + a.off)) * xr[k];
    s = block_sum256(s, red);
    const float c = __fdiv_rn(((s * ir) * ir) * ir, (float)a.d);
    for (int k = threadIdx.x; k < a.d; k += 256) {
      const float gk = dr[k] * (a.norm[k] + a.off);
      o[k] = (j == i ? 0.0f : o[k]) + (gk * ir - xr[k] * c);
    }
  }
}

// ============================================================== decoder block (model-level step)
#include "rtq_model_kernels.hip"
