// rtq_attn.hip — fused causal GQA attention of the training step (Attention::forward / backward,
// src/attention.rs:187-235, :262-320), without materialising the probabilities.  Included by
// rtq_model_kernels.hip (one code object).
//
// Arithmetic: f32 MFMA 16x16x4 (exact f32 products, f32 accumulation), as the reference's f32 dot
// products; q is scaled first (q * scale rounded, then dotted with k, as the reference orders it).
// The forward keeps, per query row, the running maximum m and sum l of exp(s - m) over the key
// tiles (a later tile with a larger maximum rescales the earlier sum and output by exp(m_old -
// m_new)); o = (sum_j exp(s_j - m) v_j) / l and lse = m + log l.  The backward recomputes
// p = exp(s - lse), dp = dO . v, ds = (p (dp - D)) scale with D = dO . o (= sum_j p_j dp_j, the
// reference's running sum), dq = sum_j ds k_j, dk = sum ds q, dv = sum p dO.  Only pairs that may
// attend enter (causal; packed layouts: the segment rule and the 64 x 64 block liveness map).
//
// Work: one wave per item (MAttnItem), four independent waves per workgroup, no barriers.  The
// operands stream from L2 straight into MFMA operand registers: an MFMA step's k slot g of lane
// (row li, g) takes contraction index 16 s + 4 g + u over the step's four MFMAs u, so a lane's
// operands of four consecutive MFMAs are one 16-byte load when the contraction index is a row's
// unit-stride index (q, k, v and dO rows over head_dim); over keys or queries (p . v, ds . k,
// p^T . dO, ds^T . q) the other operand's lane reads single floats of four rows.  The MFMA output
// layout (lane = column li, rows 4 g .. 4 g + 3) of a probability / score-gradient tile is turned
// into the operand layout (lane = row li) through a per-wave 16 x 64 LDS tile.
//
// An item covering only part of its block's range writes a partial (o, m, l; dq; dk, dv) to its
// slot; rtq_m_attn_merge_* combine a block's slots in slot order (deterministic).

constexpr int kAttnLd = 68;  // LDS row stride (floats) of the per-wave 16 x 64 transpose tile

__device__ __forceinline__ float group16_max(float v) {
#pragma unroll
  for (int m = 1; m <= 8; m <<= 1) v = fmaxf(v, __shfl_xor(v, m));
  return v;
}
__device__ __forceinline__ float group16_sum(float v) {
#pragma unroll
  for (int m = 1; m <= 8; m <<= 1) v = v + __shfl_xor(v, m);
  return v;
}

// may query i attend to key j (si: segment of i)?  Rows past t attend to nothing.
__device__ __forceinline__ bool attn_ok(const MAttnArgs& a, int i, int j, int si) {
  return j <= i && i < a.t && (!a.seg || a.seg[j] == 0 || a.seg[j] == si);
}
__device__ __forceinline__ int attn_seg(const MAttnArgs& a, int i) { return a.seg ? a.seg[min(i, a.t - 1)] : 0; }
__device__ __forceinline__ bool attn_tile_live(const MAttnArgs& a, int qblk64, int kblk64) {
  return !a.live || a.live[(int64_t)qblk64 * a.nlb + kblk64];
}

// lane (row li, slot g): the 16 x HD row block of X (row stride ld, head offset) in operand order,
// xa[4 s + u] = X[row][16 s + 4 g + u] (rows past t read row t - 1), times mul
template <int HD>
__device__ __forceinline__ void attn_rows(const float* X, int64_t ld, int r0, int t, float mul, float (&xa)[HD / 4]) {
  const int lane = threadIdx.x & 63, li = lane & 15, g = lane >> 4;
  const float* p = X + (int64_t)min(r0 + li, t - 1) * ld + 4 * g;
#pragma unroll
  for (int s = 0; s < HD / 16; s++) {
    const f4 v = *reinterpret_cast<const f4*>(p + 16 * s);
#pragma unroll
    for (int u = 0; u < 4; u++) xa[4 * s + u] = mul == 1.0f ? v[u] : v[u] * mul;
  }
}

// the four 16-column MFMA tiles of A_rows . B^T over head_dim: acc[j] += sum_e xa[e] B[r0 + 16 j + li][e]
// (B rows at stride ld from base, rows past t read row t - 1), times bmul for B (1: as stored)
template <int HD>
__device__ __forceinline__ void attn_qk(const float (&xa)[HD / 4], const float* base, int64_t ld, int c0, int t,
                                        float bmul, f4 (&acc)[4]) {
  const int lane = threadIdx.x & 63, li = lane & 15, g = lane >> 4;
  const float* rows[4];
#pragma unroll
  for (int j = 0; j < 4; j++) rows[j] = base + (int64_t)min(c0 + 16 * j + li, t - 1) * ld + 4 * g;
#pragma unroll
  for (int s = 0; s < HD / 16; s++) {
    f4 b[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      b[j] = *reinterpret_cast<const f4*>(rows[j] + 16 * s);
      if (bmul != 1.0f) b[j] = b[j] * bmul;
    }
#pragma unroll
    for (int u = 0; u < 4; u++)
#pragma unroll
      for (int j = 0; j < 4; j++) acc[j] = mfma_f32(xa[4 * s + u], b[j][u], acc[j]);
  }
}

// acc[c] (16 rows x HD) += T . Y where the 16 x 64 tile T is in MFMA output order in tv[j][i] (row
// 4 g + i, column 16 j + li) and Y's rows are r0 .. r0 + 63 (stride ld, rows past t read row t - 1):
// T goes through the wave's LDS tile sc into operand order first
template <int HD>
__device__ __forceinline__ void attn_tile_times_rows(const float (&tv)[4][4], float* sc, const float* Y, int64_t ld,
                                                     int r0, int t, f4 (&acc)[HD / 16]) {
  const int lane = threadIdx.x & 63, li = lane & 15, g = lane >> 4;
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) sc[(4 * g + i) * kAttnLd + 16 * j + li] = tv[j][i];
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int s = 0; s < 4; s++) {
    const f4 ta = *reinterpret_cast<const f4*>(sc + li * kAttnLd + 16 * s + 4 * g);
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const float* yr = Y + (int64_t)min(r0 + 16 * s + 4 * g + u, t - 1) * ld + li;
#pragma unroll
      for (int c = 0; c < HD / 16; c++) acc[c] = mfma_f32(ta[u], yr[16 * c], acc[c]);
    }
  }
  __builtin_amdgcn_wave_barrier();
}

// ------------------------------------------------------------------ forward
template <int HD>
__device__ __forceinline__ void attn_fwd_item(const MAttnArgs& a, const MAttnItem& it, float* sc) {
  constexpr int NC = HD / 16;
  const int lane = threadIdx.x & 63, li = lane & 15, g = lane >> 4;
  const int h = it.head, kvh = h / (a.nh / a.nkv), r0 = it.blk * 16;
  float qa[HD / 4];
  attn_rows<HD>(a.q + (int64_t)h * HD, a.ldq, r0, a.t, a.scale, qa);
  int si[4];
#pragma unroll
  for (int i = 0; i < 4; i++) si[i] = attn_seg(a, r0 + 4 * g + i);
  const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  f4 oacc[NC];
#pragma unroll
  for (int c = 0; c < NC; c++) oacc[c] = zero;
  float mr[4], lr[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    mr[i] = -__builtin_inff();
    lr[i] = 0.0f;
  }
  const float* kb = a.k + (int64_t)kvh * HD;
  const float* vb = a.v + (int64_t)kvh * HD;
  for (int kt = it.b0; kt < it.b1; kt++) {
    if (!attn_tile_live(a, r0 >> 6, kt)) continue;
    const int k0 = kt * 64;
    f4 s[4] = {zero, zero, zero, zero};
    attn_qk<HD>(qa, kb, a.ldk, k0, a.t, 1.0f, s);
    float p[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int row = r0 + 4 * g + i;
      float mx = -__builtin_inff();
#pragma unroll
      for (int j = 0; j < 4; j++) {
        p[j][i] = attn_ok(a, row, k0 + 16 * j + li, si[i]) ? s[j][i] : -__builtin_inff();
        mx = fmaxf(mx, p[j][i]);
      }
      mx = group16_max(mx);
      const float mn = fmaxf(mr[i], mx);
      const float corr = mr[i] == -__builtin_inff() ? 0.0f : expf(mr[i] - mn);
      float ls = 0.0f;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        p[j][i] = p[j][i] == -__builtin_inff() ? 0.0f : expf(p[j][i] - mn);
        ls = ls + p[j][i];
      }
      ls = group16_sum(ls);
      lr[i] = lr[i] * corr + ls;
      mr[i] = mn;
#pragma unroll
      for (int c = 0; c < NC; c++) oacc[c][i] = oacc[c][i] * corr;
    }
    attn_tile_times_rows<HD>(p, sc, vb, a.ldv, k0, a.t, oacc);
  }
  if (it.slot < 0) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int row = r0 + 4 * g + i;
      if (row >= a.t) continue;
      float* orow = a.o + (int64_t)row * a.ldq + (int64_t)h * HD + li;
#pragma unroll
      for (int c = 0; c < NC; c++) orow[16 * c] = __fdiv_rn(oacc[c][i], lr[i]);
      if (li == 0) a.lse[(int64_t)h * a.t + row] = mr[i] + logf(lr[i]);
    }
  } else {
    float* pp = a.part + (int64_t)it.slot * (32 * HD);
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
      for (int c = 0; c < NC; c++) pp[(4 * g + i) * HD + 16 * c + li] = oacc[c][i];
      if (li == 0) {
        pp[16 * HD + 4 * g + i] = mr[i];
        pp[16 * HD + 16 + 4 * g + i] = lr[i];
      }
    }
  }
}

// a block's partials (o, m, l) combined in slot order: m* = max m_s, l* = sum l_s exp(m_s - m*),
// o = (sum o_s exp(m_s - m*)) / l*, lse = m* + log l*; one thread per output element e of the
// 16 x hd block (its row's m*, l* recomputed by each thread of the row)
__device__ __forceinline__ void attn_merge_fwd(const MAttnArgs& a, const MAttnMerge& mg, int e) {
  const int HD = a.hd, rl = e / HD, c = e % HD, row = mg.blk * 16 + rl;
  if (row >= a.t) return;
  const float* p0 = a.part + (int64_t)mg.s0 * (32 * HD);
  float m = -__builtin_inff();
  for (int s = 0; s < mg.n; s++) m = fmaxf(m, p0[(int64_t)s * 32 * HD + 16 * HD + rl]);
  float l = 0.0f, o = 0.0f;
  for (int s = 0; s < mg.n; s++) {
    const float* ps = p0 + (int64_t)s * 32 * HD;
    const float ms = ps[16 * HD + rl];
    if (ms == -__builtin_inff()) continue;
    const float w = expf(ms - m);
    l = l + ps[16 * HD + 16 + rl] * w;
    o = o + ps[rl * HD + c] * w;
  }
  a.o[(int64_t)row * a.ldq + (int64_t)mg.head * HD + c] = __fdiv_rn(o, l);
  if (c == 0) a.lse[(int64_t)mg.head * a.t + row] = m + logf(l);
}

// ------------------------------------------------------------------ backward
// D[h][i] = sum_e dO[i][h][e] o[i][h][e]: one wave per (query, head)
__device__ __forceinline__ void attn_bwd_d(const MAttnArgs& a) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= (int64_t)a.t * a.nh) return;
  const int i = (int)(r / a.nh), h = (int)(r % a.nh);
  const float* d = a.dO + (int64_t)i * a.ldq + (int64_t)h * a.hd;
  const float* o = a.o + (int64_t)i * a.ldq + (int64_t)h * a.hd;
  float s = 0.0f;
  for (int e = lane; e < a.hd; e += 64) s = s + d[e] * o[e];
  s = wave_sum(s);
  if (lane == 0) a.D[(int64_t)h * a.t + i] = s;
}

// dq of a 16-row query block over the item's key tiles
template <int HD>
__device__ __forceinline__ void attn_dq_item(const MAttnArgs& a, const MAttnItem& it, float* sc) {
  constexpr int NC = HD / 16;
  const int lane = threadIdx.x & 63, li = lane & 15, g = lane >> 4;
  const int h = it.head, kvh = h / (a.nh / a.nkv), r0 = it.blk * 16;
  float qa[HD / 4], da[HD / 4];
  attn_rows<HD>(a.q + (int64_t)h * HD, a.ldq, r0, a.t, a.scale, qa);
  attn_rows<HD>(a.dO + (int64_t)h * HD, a.ldq, r0, a.t, 1.0f, da);
  int si[4];
  float lq[4], Dq[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int row = min(r0 + 4 * g + i, a.t - 1);
    si[i] = attn_seg(a, row);
    lq[i] = a.lse[(int64_t)h * a.t + row];
    Dq[i] = a.D[(int64_t)h * a.t + row];
  }
  const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  f4 acc[NC];
#pragma unroll
  for (int c = 0; c < NC; c++) acc[c] = zero;
  const float* kb = a.k + (int64_t)kvh * HD;
  const float* vb = a.v + (int64_t)kvh * HD;
  for (int kt = it.b0; kt < it.b1; kt++) {
    if (!attn_tile_live(a, r0 >> 6, kt)) continue;
    const int k0 = kt * 64;
    f4 s[4] = {zero, zero, zero, zero}, dp[4] = {zero, zero, zero, zero};
    attn_qk<HD>(qa, kb, a.ldk, k0, a.t, 1.0f, s);
    attn_qk<HD>(da, vb, a.ldv, k0, a.t, 1.0f, dp);
    float ds[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const bool ok = attn_ok(a, r0 + 4 * g + i, k0 + 16 * j + li, si[i]);
        const float p = expf(s[j][i] - lq[i]);
        ds[j][i] = ok ? (p * (dp[j][i] - Dq[i])) * a.scale : 0.0f;
      }
    attn_tile_times_rows<HD>(ds, sc, kb, a.ldk, k0, a.t, acc);
  }
  if (it.slot < 0) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int row = r0 + 4 * g + i;
      if (row >= a.t) continue;
      float* q = a.dq + (int64_t)row * a.ldq + (int64_t)h * HD + li;
#pragma unroll
      for (int c = 0; c < NC; c++) q[16 * c] = acc[c][i];
    }
  } else {
    float* pp = a.part + (int64_t)it.slot * (32 * HD);
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int c = 0; c < NC; c++) pp[(4 * g + i) * HD + 16 * c + li] = acc[c][i];
  }
}

// dk, dv of a 16-key block of KV head it.head over the item's (group head, query tile) pairs
template <int HD>
__device__ __forceinline__ void attn_dkv_item(const MAttnArgs& a, const MAttnItem& it, float* sc) {
  constexpr int NC = HD / 16;
  const int lane = threadIdx.x & 63, li = lane & 15, g = lane >> 4;
  const int kvh = it.head, grp = a.nh / a.nkv, c0 = it.blk * 16, nqt = (a.t + 63) / 64;
  float ka[HD / 4], va[HD / 4];
  attn_rows<HD>(a.k + (int64_t)kvh * HD, a.ldk, c0, a.t, 1.0f, ka);
  attn_rows<HD>(a.v + (int64_t)kvh * HD, a.ldv, c0, a.t, 1.0f, va);
  const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  f4 dk[NC], dv[NC];
#pragma unroll
  for (int c = 0; c < NC; c++) dk[c] = dv[c] = zero;
  for (int pr = it.b0; pr < it.b1; pr++) {
    const int h = kvh * grp + pr / nqt, qt = pr % nqt, q0 = qt * 64;
    if (q0 + 63 < c0 || !attn_tile_live(a, qt, c0 >> 6)) continue;
    const float* qh = a.q + (int64_t)h * HD;
    const float* dh = a.dO + (int64_t)h * HD;
    f4 st[4] = {zero, zero, zero, zero}, dpt[4] = {zero, zero, zero, zero};
    attn_qk<HD>(ka, qh, a.ldq, q0, a.t, a.scale, st);  // S^T: keys x queries, q scaled as stored order
    attn_qk<HD>(va, dh, a.ldq, q0, a.t, 1.0f, dpt);    // dP^T = V dO^T
    float pt[4][4], dst[4][4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int qr = q0 + 16 * j + li, qc = min(qr, a.t - 1);
      const float lq = a.lse[(int64_t)h * a.t + qc], Dq = a.D[(int64_t)h * a.t + qc];
      const int sq = attn_seg(a, qc);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const bool ok = attn_ok(a, qr, c0 + 4 * g + i, sq);
        const float p = ok ? expf(st[j][i] - lq) : 0.0f;
        pt[j][i] = p;
        dst[j][i] = ok ? (p * (dpt[j][i] - Dq)) * a.scale : 0.0f;
      }
    }
    attn_tile_times_rows<HD>(pt, sc, dh, a.ldq, q0, a.t, dv);   // dV += P^T dO
    attn_tile_times_rows<HD>(dst, sc, qh, a.ldq, q0, a.t, dk);  // dK += dS^T Q
  }
  if (it.slot < 0) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int key = c0 + 4 * g + i;
      if (key >= a.t) continue;
      float* kr = a.dk + (int64_t)key * a.ldk + (int64_t)kvh * HD + li;
      float* vr = a.dv + (int64_t)key * a.ld_dv + (int64_t)kvh * HD + li;
#pragma unroll
      for (int c = 0; c < NC; c++) {
        kr[16 * c] = dk[c][i];
        vr[16 * c] = dv[c][i];
      }
    }
  } else {
    float* pp = a.part + (int64_t)it.slot * (32 * HD);
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int c = 0; c < NC; c++) {
        pp[(4 * g + i) * HD + 16 * c + li] = dk[c][i];
        pp[16 * HD + (4 * g + i) * HD + 16 * c + li] = dv[c][i];
      }
  }
}

// sums of a block's partials in slot order, one thread per element e: dq (kv = false, 16 x hd) or
// dk then dv (kv = true, 2 x 16 x hd)
__device__ __forceinline__ void attn_merge_sum(const MAttnArgs& a, const MAttnMerge& mg, int e, bool kv) {
  const int HD = a.hd;
  const int part = e / (16 * HD), rl = (e % (16 * HD)) / HD, c = e % HD, row = mg.blk * 16 + rl;
  if (row >= a.t) return;
  const float* p0 = a.part + (int64_t)mg.s0 * (32 * HD) + e;
  float s = 0.0f;
  for (int k = 0; k < mg.n; k++) s = s + p0[(int64_t)k * 32 * HD];
  if (!kv)
    a.dq[(int64_t)row * a.ldq + (int64_t)mg.head * HD + c] = s;
  else if (part == 0)
    a.dk[(int64_t)row * a.ldk + (int64_t)mg.head * HD + c] = s;
  else
    a.dv[(int64_t)row * a.ld_dv + (int64_t)mg.head * HD + c] = s;
}

// ------------------------------------------------------------------ entry points (grid: ceil(n / 4) x 256)
#define RTQ_ATTN_ITEM_KERNEL(NAME, FN, HD)                                             \
  extern "C" __global__ __launch_bounds__(256) void NAME(MAttnArgs a) {                \
    __shared__ __attribute__((aligned(16))) float sc[4][16 * kAttnLd];                 \
    const int id = blockIdx.x * 4 + (threadIdx.x >> 6);                                \
    if (id >= a.n_items) return; /* whole wave; waves never wait on each other */      \
    FN<HD>(a, a.items[id], sc[threadIdx.x >> 6]);                                      \
  }
RTQ_ATTN_ITEM_KERNEL(rtq_m_attn_fwd64, attn_fwd_item, 64)
RTQ_ATTN_ITEM_KERNEL(rtq_m_attn_fwd128, attn_fwd_item, 128)
RTQ_ATTN_ITEM_KERNEL(rtq_m_attn_dq64, attn_dq_item, 64)
RTQ_ATTN_ITEM_KERNEL(rtq_m_attn_dq128, attn_dq_item, 128)
RTQ_ATTN_ITEM_KERNEL(rtq_m_attn_dkv64, attn_dkv_item, 64)
RTQ_ATTN_ITEM_KERNEL(rtq_m_attn_dkv128, attn_dkv_item, 128)
#undef RTQ_ATTN_ITEM_KERNEL

// merges: grid n_merges x ceil(elements / 256) (flat), one thread per element of a block
#define RTQ_ATTN_MERGE_KERNEL(NAME, NEL, CALL)                                          \
  extern "C" __global__ __launch_bounds__(256) void NAME(MAttnArgs a) {                 \
    const int per = (NEL + 255) / 256, mi = blockIdx.x / per;                           \
    const int e = (blockIdx.x % per) * 256 + threadIdx.x;                               \
    if (mi < a.n_merges && e < NEL) CALL;                                               \
  }
RTQ_ATTN_MERGE_KERNEL(rtq_m_attn_merge_fwd, 16 * a.hd, attn_merge_fwd(a, a.merges[mi], e))
RTQ_ATTN_MERGE_KERNEL(rtq_m_attn_merge_dq, 16 * a.hd, attn_merge_sum(a, a.merges[mi], e, false))
RTQ_ATTN_MERGE_KERNEL(rtq_m_attn_merge_dkv, 32 * a.hd, attn_merge_sum(a, a.merges[mi], e, true))
#undef RTQ_ATTN_MERGE_KERNEL
extern "C" __global__ __launch_bounds__(256) void rtq_m_attn_bwd_d(MAttnArgs a) { attn_bwd_d(a); }
