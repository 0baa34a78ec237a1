// rtq_kargs.h — kernel argument blocks and device-layout constants shared by the host runtime
// (rtq_runtime.cpp) and the gfx950 kernels (rtq_kernels.hip).  Every kernel takes exactly one
// of these structs by value, so hipModuleLaunchKernel passes one parameter.
//
// Device weight layout ("row-group / K-chunk" layout, same byte count as GGUF):
//   rows are padded to Np = roundup(N, 64) and grouped by 16 (one MFMA tile edge); columns
//   are padded to Kp = roundup(K, 128) for Q4_0 / Q8_0 (a chunk = 4 blocks of 32).  For every
//   (row group rg, chunk kc) the quant codes of the 16 rows are stored so that lane l of a
//   wave (row rg*16 + l%16, k-group g = l/16) reads its MFMA fragment with one coalesced
//   load: lane l holds, for every 32-element block j of the chunk, the codes of elements
//   {32j + 4g .. 32j + 4g + 3} and {32j + 16 + 4g .. 32j + 16 + 4g + 3}.  For Q4_0 that is
//   exactly bytes 4g..4g+3 of the GGUF block (low nibbles: the first four, high nibbles: the
//   second four), so no nibble moves across bytes.
//     Q4_0: qs  uint4 [Np/16][Kc][64]      (component j = block j's four bytes)
//     Q8_0: qs  uint4 [Np/16][Kc][2][64]   (part p: blocks 2p, 2p+1; 8 bytes each: low word
//                                           elements 4g..4g+3, high word 16+4g..16+4g+3)
//     both: d   fp16  [Np/16][Kc][2 h][4 q][2 j2][4 i]   scale of row 4q+i of the group, block
//           2h+j2 of the chunk: the lane with k-group q reads the scales of rows 4q..4q+3 for
//           a half chunk (two blocks) with one 16-byte load, which is the row set a lane holds
//           in the output of an MFMA whose A operand is the weight;
//           wdr fp16 [Np/16][Kc][16 li][4 j] (RTQ_WR_INDEX): the same scales row by row, for the
//           GEMV kernel, whose lanes hold one weight row each (8 bytes per lane and chunk).
//   K-quants (256-element super-blocks, Kp = K) are transcoded at upload into the same code
//   layouts, with their 6-bit sub-block scales kept as integers:
//     Q4_K: qs as Q4_0, unsigned 4-bit codes u (value d*sc*u - dmin*m);
//     Q6_K: qs as Q8_0, signed codes q in [-32, 31] (value d*sc*q, sc per 16 elements);
//     wd (uint16) [Np/16][Kc][16 li][4 j] (RTQ_WR_INDEX): block j of row li, low byte sc (Q6_K: sc
//           of elements 0..15), high byte m (Q6_K: sc of elements 16..31, int8).  The lane that
//           builds row li's MFMA fragment reads one 32-bit word per half chunk;
//     wsb (uint32) [Np/16][Kp/256][16 li] (RTQ_WSB_INDEX): fp16 d (low) and fp16 dmin (high; 0
//           for Q6_K) of the super-block; the lane with k-group q reads rows 4q..4q+3 at once.
#pragma once
#include <stdint.h>

#define RTQ_ROW_PAD 64    // Np multiple
#define RTQ_CHUNK_Q 128   // K chunk of Q4_0 / Q8_0
#define RTQ_ACT_KQ 256    // columns per activation-prep workgroup (one LoRA-down partial each)
#define RTQ_LDS_RANK 64   // LoRA ranks up to this are staged in LDS by the forward kernels
#define RTQ_MM_RING 3     // rtq_mm_* (128 x 128 tiles): stages of the operand ring in LDS
#define RTQ_MM64_RING 3   // rtq_mm64_* (128 x 64 tiles)
#define RTQ_MM32_RING 3   // rtq_mm32_* (128 x 32 tiles)

// index of the row-major scale (K-quants: sub-block scale word) of row li of row group rg, block j
// of chunk kc
#define RTQ_WR_INDEX(rg, kc, Kc, li, j) ((((int64_t)(rg) * (Kc) + (kc)) * 16 + (li)) * 4 + (j))
// index of the K-quant super-block scale pair of row li of row group rg, super-block sb
#define RTQ_WSB_INDEX(rg, sb, Ksb, li) (((int64_t)(rg) * (Ksb) + (sb)) * 16 + (li))

// index of the fp16 scale of row li (0..15) of row group rg, block j (0..3) of chunk kc
#define RTQ_WD_INDEX(rg, kc, Kc, li, j) \
  (((((int64_t)(rg) * (Kc) + (kc)) * 2 + ((j) >> 1)) * 4 + ((li) >> 2)) * 8 + ((j) & 1) * 4 + ((li) & 3))

// ---------------------------------------------------------------- forward activation prep
// Grid (Tp/16, nhp), nhp = Kp / RTQ_ACT_KQ rounded up to a multiple of 4; workgroup (x, y)
// covers 16 tokens x columns [256y, 256y + 256) (the block-norm kernels rtq_act_prep8 / 4: 8 or 4
// tokens, grid (Tp/8 or Tp/4, nhp)).  x [T x K] f32 ->
//   xq: Q8_0 codes as exact-f16 MFMA fragments: uint4 [Tp/16][Kp/128][4][64] (8 per lane per block)
//   xd: f32 [Kp/128][Tp][4]  (value of the fp16 scale of block 4kc+j of token t; 0 for padding)
//   hp: LoRA down-projection partials [T][r][nhp] (src/linear.rs:85): partial y sums the
//       workgroup's columns; the forward GEMM sums them in order
//   zero_y: rows of y cleared when the forward GEMM splits K across workgroups (atomics)
// rtq_act_prep_q8_k (K-quant weights): Q8_K per 256-column super-block (one workgroup's
// columns), same xq layout; xd holds the super-block's f32 d for each of its 32-element blocks.
// xg (GEMV, Tp = 16): [Kp/32][2][16]: the block's scale per token, then -gbias * (sum of the
// block's codes) per token (the accumulator seed that removes the GEMV's code bias).
struct ActArgs {
  const float* x;
  int T, K, Tp, Kp;
  void* xq;
  float* xd;
  float* xg;
  float gbias;
  const float* A;
  int r;
  float* hp;
  float* zero_y;
  int N;
  uint16_t* xdh;  // or null: the fp16 bits of xd, same layout (rtq_mm_*'s scale MFMA operand)
  // or null: the activation is SwiGLU's silu(sg) * su (src/model.rs:124, rows of stride ldsg),
  // computed here and written to x (then an output) for the backward
  const float* sg;
  const float* su;
  int ldsg;
  // 1: the codes go to xq as int8 fragments of rtq_mmi8_* ([Tp/32][Kc][4][64] x 16 bytes, lane l:
  // token l % 32, the block's codes of k-groups 2 (l / 32) and 2 (l / 32) + 1), not f16 ones
  int xq_i8;
  // or null: the activation is RMSNorm of na (+ nb) (src/ops.rs:14-35) with weight nw (+ noff), in
  // the order of rtq_m_rmsnorm's one-wave rows (K % 256 == 0, K <= 1024), formed here; the rows go
  // to x (then an output), na + nb to nh (with nb), 1 / rms to ninv (rows [T])
  const float* na;
  const float* nb;
  float* nh;
  const float* nw;
  float* ninv;
  float neps, noff;
};

// ---------------------------------------------------------------- trainer-native weights
// FrozenWeight::{F32, Q8_0} (src/frozen.rs:33-45): f32 [N][K], or f32 scales [N][K/32] then i8
// codes [N][K] (TQ8_0).  Their products run on the f32 MFMA GEMM (rtq_m_gemm*, the TQ8_0 codes
// decoded in its operand loads); these kernels dequantise rows (out = 0 + d * q, row() of
// src/frozen.rs:172-176), copy rows and add the bias.
struct DenseArgs {
  const float* w;    // F32 weight, or null
  const float* sc;   // TQ8_0 scales, or null
  const int8_t* qs;  // TQ8_0 codes
  int64_t N, K;
  int64_t r0, count;  // rows [r0, r0 + count) (dequant / row copy); bias: count = T
  float* out;         // [count][K]; bias: y [T][N]
  const float* bias;
  const int32_t* idx;  // or null: out row i is weight row idx[i] (embedding gather), else r0 + i
};

// ---------------------------------------------------------------- forward GEMM
// y[t][n] = sum_b d_w[n][b] d_x[t][b] isum_b(t, n)  (+ bias[n]) (+ s * sum_j h[t][j] B[n][j])
// K-quants: sum over super-blocks of (d d_x) S1 - (dmin d_x) S2 (Q4_K) or (d d_x) S (Q6_K)
// Block-diagonal adapter of row-concatenated weights (a fused q|k|v or gate|up projection):
// member m owns weight rows [row0[m], row0[m] + nrow[m]) and ranks [col0[m], col0[m] + r[m]) (r 0:
// not adapted); only those (row, rank) pairs of B and gb exist.  nm = 0: one plain adapter.
struct RankBlocks {
  int nm;
  int row0[3], nrow[3], col0[3], r[3];
};

struct FwdArgs {
  const void* wq;       // quant codes, device layout
  const uint16_t* wd;   // fp16 scales (K-quants: sub-block scale words), device layout
  const uint16_t* wdr;  // row-major scales (RTQ_WR_INDEX; the K-quants' wd itself)
  const float* xg;      // GEMV activation scales and seeds [Kp/32][2][16]
  int Np, Kp;
  const void* xq;       // activation fragments (f16 integer codes)
  const float* xd;      // activation scales [Kp/128][Tp][4]
  const uint32_t* wsb;  // K-quant super-block scales (RTQ_WSB_INDEX)
  int Tp, T, N, K;
  int kc_per_split;     // K chunks per blockIdx.z (split-K across workgroups accumulates with atomics)
  float* y;             // [T x N]
  const float* bias;    // [N] or null
  const float* hp;      // LoRA down-projection partials [T][r][nhp] or null (LoRA disabled)
  int nhp;
  const float* lb;      // LoRA B [N x r]
  int r;
  float s;              // alpha / r
  int32_t* isums;       // debug: [T][N][K/32] (Q4_0, Q8_0), [T][N][K/256][2] (Q4_K: S1, S2),
                        // [T][N][K/256] (Q6_K: S), or null
  const uint16_t* xdh;  // fp16 activation scales, layout of xd (rtq_mm_*)
  RankBlocks rb;        // LoRA B's block structure: a row's up-projection reads its member's ranks only
};

// rtq_gemvq{1,4}_*: row groups per tile (nibble codes, byte codes) and register-ring depth
#ifndef RTQ_GQ_RG4
#define RTQ_GQ_RG4 2
#endif
#ifndef RTQ_GQ_RG8
#define RTQ_GQ_RG8 1
#endif
#ifndef RTQ_GQ_D
#define RTQ_GQ_D 4
#endif
#ifndef RTQ_DXV1_D
#define RTQ_DXV1_D 4  // rtq_dxv1_*: register ring depth (row groups; loads D - 1 ahead); 6 and 8
                      // measured slower (LM head backward at T = 1, Q4_0 24.1 -> 25.3 / 26.2 us)
#endif
#ifndef RTQ_DX16_D
#define RTQ_DX16_D 4  // rtq_dx16_*: register ring depth (steps of 32 rows; loads D - 1 steps ahead)
#endif
#ifndef RTQ_DX16_SCAN
#define RTQ_DX16_SCAN 8  // rtq_dx16_*: float4 loads in flight per thread in the dy range scan
#endif
// rtq_gemvq{1,4}_*: y = x W^T (+ bias) (+ s (x A^T) B^T) for T <= 1 / 4 tokens in one launch (the
// kernel quantises x itself).  Dynamic LDS: NT Kp bytes of codes, NT Kp / 32 block scales, NT Kp / 32
// code sums (Q4_0: NT Kp / 8, one per k-group), NT * RTQ_LDS_RANK floats of h.
struct GemvqArgs {
  const void* wq;
  const uint16_t* wdr;  // row-major scales (RTQ_WR_INDEX; the K-quants' sub-block scale words)
  const uint32_t* wsb;  // K-quant super-block scales (RTQ_WSB_INDEX)
  int Np, Kp;
  const float* x;       // [T x K]
  int T, N, K;
  float* y;             // [T x N]
  const float* bias;    // [N] or null
  const float* la;      // LoRA A [r x K], or null (no adapter)
  const float* lb;      // LoRA B [N x r]
  int r;
  float s;
  RankBlocks rb;
  int ntiles;           // row tiles of the weight (its row groups in runs of the kernel's RG)
  int tiles_per_wave;   // wave v takes tiles v, v + waves, ... (at most this many)
};

// ---------------------------------------------------------------- backward
// rtq_bwd_prep: partials of h = x . A^T and of dy . B per 256-column slice (src/linear.rs:106-111)
struct BwdPrepArgs {
  const float* x;
  const float* A;
  int K;
  const float* dy;
  const float* B;
  int N;
  int T, r;
  float* hp;     // [T][r][nhq] partials of x . A^T
  int nhq;
  float* gp;     // [ngq][T][r] partials of dy . B
  int ngq;
  float* dymax;  // [ngq][T]: max |dy| over each 256-row slice (the dx kernels' f16 range), or null
  RankBlocks rb;  // g = dy . B restricted to each member's rows
  int y0;         // grid row offset: nhq when the h partials are already there (only g is computed)
  int gtok;       // tokens per g-partial workgroup: 64 (a wave per 16 tokens), 32 (a wave per 16 tokens
                  // and 128 rows) or 16 (a wave per 64 rows)
};

// part[z][t][k] = sum over rows n of split z of dy[t][n] W[n][k], three 16-bit MFMAs per product (hi / lo
// split of dy and W: f16 with dy scaled per row by rtq_dx_* / rtq_dxw_*, bf16 by rtq_dx16_*).
// rtq_dx_*: workgroup tile 64 tokens x 128 columns, partials in MFMA fragment order; rtq_dx16_*
// (T <= 16): tile 16 tokens x 128 columns, partials row-major [nsplit][T][K].
struct DxArgs {
  const void* wq;
  const uint16_t* wd;
  const uint32_t* wsb;  // K-quant super-block scales (RTQ_WSB_INDEX)
  int Np, Kp;
  const float* dy;
  int T, N, K;
  int n_per_split;      // rows of W per split (multiple of 32)
  int nsplit;           // splits: grid = Kc * ceil(T/64) * nsplit workgroups (+ LoRA finalisers)
  float* part;          // [splits][T][K] partial products
  // LoRA finalisation by the extra workgroups of the last grid row (when gp != null):
  const float* hp;      // [T][r][nhq] partials from rtq_bwd_prep
  const float* gp;      // [ngq][T][r]
  int nhq, ngq, r;
  float s;
  float* h;             // [T x r] = sum of hp
  float* g;             // [T x r] = s * sum of gp
  // rtq_dx_* / rtq_dxw_*: f16 operands need dy's range: dymax [dmq][T] = max |dy[t][n]| over the
  // 256-row slice q (rtq_bwd_prep); W's values scaled by wsc = 2^-sigma, the partials by wunsc
  const float* dymax;
  int dmq;
  float wsc, wunsc;
  const uint16_t* wdr;  // row-major scales (RTQ_WR_INDEX): rtq_dxv1_*
};

// dx[t][k] = [dx +] sum_s part[s][t][k] [+ sum_j g[t][j] A[j][k]];
// gb[n][j] += sum_t (s*dy[t][n]) h[t][j];  ga[j][k] += sum_t g[t][j] x[t][k]
struct LoraGradArgs {
  const float* dy;
  const float* h;
  const float* g;       // null: no LoRA
  const float* x;
  const float* la;
  int T, N, K, r;
  float s;
  float* gb;  // [N x r]
  float* ga;  // [r x K]
  float* dx;  // [T x K]
  int n_gb, n_ga, n_dx;  // workgroups of each part, in this order
  const float* part;     // split partials from the dx kernel
  int nsplit;
  int accumulate;        // 1: dx += (FrozenMatmul::backward_input); 0: dx = (Linear::backward)
  int part_rows;         // 1: partials row-major [nsplit][T][K] (rtq_dx16_*); 0: fragment order (rtq_dx_*)
  RankBlocks rb;         // gb written only inside the members' blocks
  // or null: dx is SwiGLU's dh (src/model.rs:126-131) and is not stored; dg = (dh u) silu'(g) and
  // du = dh silu(g) go to swdg / swdu instead (g, u, dg, du: rows of stride swld)
  const float* swg;
  const float* swu;
  float* swdg;
  float* swdu;
  int64_t swld;
  int sw_keep;  // 1: dh is stored to dx as well (a layer whose activations are being captured)
};

// dA / dB of up to RTQ_LORA_JOBS linears in one launch (rtq_lora_grads[16]): workgroups
// [start[j], start[j + 1]) are job j's gb tiles (its n_gb) then its ga tiles (n_ga) of 64 rows
#define RTQ_LORA_JOBS 8
struct LoraGradBatch {
  int njobs;
  int start[RTQ_LORA_JOBS + 1];
  LoraGradArgs job[RTQ_LORA_JOBS];
};

// dA / dB tiles of any number of linears from a job table in device memory (rtq_lora_grads_t[16]):
// workgroup b runs tile map[2 b + 1] of job map[2 b] (its gb tiles, then its ga tiles)
struct LoraGradTable {
  const LoraGradArgs* job;
  const int* map;
};

// rows [r0, r0+count) dequantised to f32 (bit-exact ggml dequant)
struct RowArgs {
  const void* wq;
  const uint16_t* wd;
  const uint32_t* wsb;
  int Np, Kp, K;
  int r0, count;
  float* out;          // [count x K]
  const int32_t* idx;  // or null: row i of out is weight row idx[i] (embedding gather), else r0 + i
  int rows;            // weight rows (bound of idx)
};

struct FillArgs {
  float* p;
  int64_t n;
};

// ---------------------------------------------------------------- LM head + cross-entropy
// Model::head (src/model.rs:561-609): final RMSNorm of the target rows, log-softmax with an f64
// normaliser (softmax_row, src/ops.rs:238-247), dlogits = w (softmax - onehot), and the RMSNorm
// backward (src/ops.rs:39-56) of dlogits . W, added into dx at the target positions.
struct HeadArgs {
  const float* x;      // [t x d] final hidden states
  const int32_t* pos;  // [n] target positions
  const int32_t* tok;  // [n] target tokens
  const float* wts;    // [n] loss weights, or null (log-probs only)
  const float* norm;   // [d] final norm weight
  float eps, off;
  int t, d, n, V;
  int G, L;            // vocabulary slices per row (grid x of the softmax kernels) and slice length
  float* ns;           // [n x d] normalised target rows (the lm_head input)
  float* inv;          // [n] 1 / rms
  float* logits;       // [n x V] logits; overwritten by dlogits when wts
  float* pmax;         // [n x G] slice maxima
  double* psum;        // [n x G] slice sums of exp(v - max)
  float* logp;         // [n]
  int32_t* hit;        // [n] 1 if the target's logit is >= every logit of its row
  const float* dns;    // [n x d] dlogits . W (lm_head backward_input)
  float* dx;           // [t x d] dL/dx (rows without a target are cleared separately)
};

// ---------------------------------------------------------------- model-level step
// The decoder block around the frozen linears (src/model.rs:165-197, src/attention.rs:162-367,
// src/model.rs:113-134, src/ops.rs:14-56, :118-196), all tensors row-major f32 on the device.
struct MNormArgs {
  const float* a;    // [rows x d] input (the residual stream)
  const float* b;    // or null: the input is a + b, written to h
  float* h;          // [rows x d] a + b (when b), else unused
  const float* w;    // [d] norm weight
  float* y;          // [rows x d]
  float* inv;        // [rows] 1 / rms
  int rows, d;
  float eps, off;
  int fused;         // 1: x * (ir * (w + off)) (QK-norm order), 0: (x * ir) * (w + off)
  int wave;          // 1: one wave per row, one-wave workgroups (d % 256 == 0, d <= 2048, 16-byte aligned rows)
};

struct MNormBwdArgs {
  const float* x;    // [rows x d] the norm's input
  const float* w;
  const float* inv;
  const float* dy;   // [rows x d] gradient of the norm's output
  const float* res;  // or null: out = res + dx_norm (the residual branch's gradient)
  float* out;        // [rows x d]
  int rows, d;
  float off;
  int wave;          // as MNormArgs::wave
};

// per (token, head) row of width hd: QK-norm, RoPE, f16 rounding of K and V
struct MAttnMerge;
struct MQkArgs {
  const float* q_raw;  // [t x nh x hd]
  const float* k_raw;  // [t x nkv x hd]
  const float* v_raw;  // [t x nkv x hd]
  const float* q_norm; // [hd] or null
  const float* k_norm;
  const float* cos_;   // [t x rot/2]
  const float* sin_;
  float* q;            // outputs, same layouts
  float* k;
  float* v;
  float* q_inv;        // [t x nh]
  float* k_inv;        // [t x nkv]
  // backward: gradients in (dq [t x nh x hd], dk), out (dq_raw, dk_raw); dv passes through
  const float* dq;
  const float* dk;
  float* dq_raw;
  float* dk_raw;
  int t, nh, nkv, hd, rot, neox, kv_f16;
  float eps, off;
  int64_t ldq, ldk, ldv;  // per-token row strides of q_raw / dq_raw, k_raw / dk_raw, v_raw (fused q|k|v rows)
  int half;               // 1: hd = rot = 128, a half-wave (32 lanes x 4 elements) per row, 8 rows per workgroup
  // backward, half-wave rows: the fused attention's partial slots of cut blocks summed here (in slot
  // order, as rtq_m_attn_merge_bwd) instead of by a merge launch; qmi null: dq, dk, dv are whole
  const int* qmi;                   // [nh x nb16]: index into qmerges of (head, 16-row block), or -1
  const int* kmi;                   // [nkv x nb16]: into kmerges (dk slots, then dv at + 16 x 128)
  const MAttnMerge* qmerges;
  const MAttnMerge* kmerges;
  const float* qpart;               // slots of 32 x 128 floats
  const float* kpart;
  float* dv;                        // merged dv rows of cut blocks, row stride ld_dv
  int64_t ld_dv;
  int nb16;
};

// C(b, m, n) (+)= sum_k A(b, m, k) * B(b, k, n), A(b, m, k) = A[(b / divA) * sAb + m * sAm + k * sAk]
// (rounded product a_scale * A first when a_scale != 1), likewise B and C.
// causal 0: full; 1: only tiles touching n <= m (others skipped); 2: k < min(K, m0 + 64) (A zero
// above the diagonal); 3: k >= m0 (A(b, m, k) zero for k < m).
// live (or null): attention layout of a packed batch, one byte per 64 x 64 block of (query i, key
// j) pairs, nonzero when some pair of the block may attend; nlb blocks per side.  The causal mode
// names the roles: 1 (m, n) = (i, j), 2 (m, k) = (i, j), 3 (m, k) = (j, i).  Dead output tiles are
// skipped (not written), dead k slabs are not read.
struct MGemmArgs {
  const float* A;
  const float* B;
  float* C;
  int M, N, K;
  int64_t sAb, sAm, sAk, sBb, sBk, sBn, sCb, sCm, sCn;
  int divA, divB;
  float a_scale;
  int causal, accumulate;
  int batch;
  const uint8_t* live;
  int nlb;
  // rtq_m_gemm*_q8: B holds int8 codes (element (k, n) at ((const int8_t*)B)[k * sBk + n * sBn]) with
  // an f32 scale per 32 consecutive codes, Bsc[code index / 32] (FrozenWeight::Q8_0, src/frozen.rs:38-45)
  const float* Bsc;
};

// up to three independent products in one launch of the 32-row-tile kernel: flat workgroup ids
// [start[i], start[i + 1]) belong to product i (column tiles fastest, then row tiles, then batch)
struct MGemmGroupArgs {
  MGemmArgs p[3];
  int np;
  int start[4];
};

// attention rows (h, i) of S / P / dP [nh x t x t]
struct MSoftArgs {
  float* s;          // forward: scores in, probabilities out (0 for j > i)
  const float* p;    // backward: probabilities
  float* dp;         // backward: dP in, dS = P (dP - sum P dP) scale out (0 for j > i)
  int t, nh;
  float scale;
  // packed layout (or null): segment of each token (j may be seen by i when seg[j] == 0 or
  // seg[j] == seg[i]) and the 64 x 64 block liveness map of MGemmArgs; only live blocks are read
  // and written (0 where a pair may not attend)
  const int32_t* seg;
  const uint8_t* live;
  int nlb;
};

// ---------------------------------------------------------------- fused attention
// One work item = one wave: (head, 16-row block of queries, range of 64-key tiles) for the
// forward and dQ passes; (KV head, 16-key block, range of (group head, 64-query tile) pairs
// p = head_in_group * ceil(t / 64) + tile) for the dK / dV pass.  slot >= 0: the item covers part
// of its block's range and writes a partial to part[slot] (merged by rtq_m_attn_merge in slot
// order); slot < 0: it covers the whole range and writes the result.  pad0: the number of items
// of the item's block.  rbase, rlen: the item's sequence is rows [rbase, rbase + rlen) of q, k,
// v, o (and columns of lse): the whole step (0, t), or, for the forward of a packed layout, one
// segment's logical sequence gathered to those rows (MSeqArgs); blk and b0, b1 count from rbase.
struct MAttnItem {
  int head, blk, b0, b1, slot, pad0, rbase, rlen;
};
// one block whose items wrote partials to slots [s0, s0 + n); rbase, rlen as its items'
struct MAttnMerge {
  int head, blk, s0, n, rbase, rlen;
};
// the forward attention of a packed layout runs over each segment's logical sequence: the rows
// whose segment is 0 or that segment, in packed order (for segment 0, its rows alone), gathered
// to back-to-back runs of rows that start at multiples of 64 (Rope::allowed, src/ops.rs:158-164:
// a row attends to exactly the earlier rows of its sequence, so each key tile covers the same
// logical positions as in the example's own run).  gather: q, k, v rows gmap[r] (-1: zero) to
// row r of gq, gk, gv for r < tv; scatter: each packed row i's own copy, row sidx[i] of go (and of
// glse, when not null), back to o (lse).
struct MSeqArgs {
  const float* q;    // packed [t][nh][hd] (ldq)
  const float* k;    // [t][nkv][hd] (ldk)
  const float* v;    // (ldv)
  float* gq;         // gathered [tv][nh][hd] (row stride nh hd), gk, gv [tv][nkv][hd]
  float* gk;
  float* gv;
  const float* go;   // gathered output [tv][nh][hd], log-sum-exp [nh][tv] (or null)
  const float* glse;
  float* o;          // packed output (ldq), lse [nh][t]
  float* lse;
  const int32_t* gmap;  // [tv]
  const int32_t* sidx;  // [t]
  int t, tv, nh, nkv, hd;
  int64_t ldq, ldk, ldv;
};
struct MAttnArgs {
  const float* q;   // [t][nh][hd] (rotated, row stride ldq)
  const float* k;   // [t][nkv][hd] (ldk)
  const float* v;   // [t][nkv][hd] (ldv)
  float* o;         // forward output [t][nh][hd] (ldq)
  float* lse;       // [nh][t]: log-sum-exp of each query row's scaled scores (forward out, backward in)
  const float* dO;  // backward: gradient of o [t][nh][hd] (ldq)
  float* D;         // backward: [nh][t], sum_e dO * o per query row
  float* dq;        // [t][nh][hd] (ldq)
  float* dk;        // [t][nkv][hd] (ldk)
  float* dv;        // rows at ld_dv
  float* part;      // partial slots
  const MAttnItem* items;
  const MAttnMerge* merges;
  int n_items, n_merges;
  // the backward's second item kind (dk, dv: items2, their partial slots part2, merges2), run in
  // the same launch as the dq items (rtq_m_fa_bwd*) and merged in the same launch
  const MAttnItem* items2;
  const MAttnMerge* merges2;
  float* part2;
  int n_items2, n_merges2;
  const int32_t* seg;  // packed layout (or null): segment per token
  const uint8_t* live; // and the 64 x 64 block liveness map (nlb blocks per side)
  int nlb;
  int t, nh, nkv, hd;
  int64_t ldq, ldk, ldv, ld_dv;
  float scale;
  // the fused backward's 16-bit operand planes, formed once per layer by rtq_m_attn_bwd_prep*:
  // natural [t][heads][hd]: q scale log2(e) (f16 hi / lo), dO (bf16 hi / lo), k (f16), v (bf16
  // hi / lo); transposed [heads][hd][tp] (tp = t rounded up to 64, columns past t zero): q, dO, k
  // (bf16 hi / lo)
  uint16_t *pqsh, *pqsl, *pdoh, *pdol, *pkf, *pvh, *pvl, *pqth, *pqtl, *pdth, *pdtl, *pkth, *pktl;
  int tp;
};

struct MGroupArgs {
  const float* dkh;  // [nh x t x hd] per-head gradients
  const float* dvh;
  float* dk;         // [t x nkv x hd]: sum of the group's heads, in head order
  float* dv;         // token i's row at dv + i * ldv
  int t, nh, nkv, hd;
  int64_t ldv;
};

// elementwise over rows x cols: a, b at row stride lda, c at ldc, y, z at ldy
struct MEltArgs {
  const float* a;
  const float* b;
  const float* c;
  float* y;
  float* z;
  int64_t n, cols, lda, ldc, ldy;
};

// clears the off-block entries of a fused adapter's gb [rows x rank]: row range m (row0[m], rows[m])
// keeps columns [col0[m], col0[m] + r[m]) only
struct MMaskArgs {
  float* gb;
  int64_t rows, rank;
  int nm;
  int64_t row0[3], nrow[3], col0[3], r[3];
};
