// rtq_attn.hip — pieces of the fused causal GQA attention of the training step (Attention::forward /
// backward, src/attention.rs:187-235, :262-320) shared by the kernels of rtq_fa.hip: the mask
// (causal; packed layouts: the segment rule and the 64 x 64 block liveness map), lane-group
// reductions, and the merges of the partials that items covering part of
// a block's range leave in slots: a 16-row block's slots combined in slot order (deterministic).
// Included by rtq_model_kernels.hip (one code object).

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

// ------------------------------------------------------------------ forward
constexpr int kMergeBatch = 8;  // merges of up to this many slots issue all their loads at once

// a block's partials (o, m, l; m a base-2 maximum) combined in slot order: m* = max m_s,
// l* = sum l_s 2^(m_s - m*), o = (sum o_s 2^(m_s - m*)) / l*, lse = m* ln 2 + log l*; one thread per
// four consecutive output elements 4 e4 .. of the 16 x hd block (its row's m*, l* recomputed by
// each thread of the row)
__device__ __forceinline__ void attn_merge_fwd(const MAttnArgs& a, const MAttnMerge& mg, int e4) {
  const int HD = a.hd, rl = 4 * e4 / HD, c = 4 * e4 % HD, row = mg.blk * 16 + rl;
  if (row >= mg.rlen) return;  // rows of the block's sequence (rbase, rlen: MAttnItem)
  const float* p0 = a.part + (int64_t)mg.s0 * (32 * HD);
  float m = -__builtin_inff(), l = 0.0f;
  f4 o = {0.0f, 0.0f, 0.0f, 0.0f};
  if (mg.n <= kMergeBatch) {  // every slot's loads issued together, then the same arithmetic in slot order
    float mv[kMergeBatch], lv[kMergeBatch];
    f4 ov[kMergeBatch];
#pragma unroll
    for (int s = 0; s < kMergeBatch; s++) {  // (n is uniform: the slots past it are not read)
      const float* ps = p0 + (int64_t)s * 32 * HD;
      mv[s] = s < mg.n ? ps[16 * HD + rl] : -__builtin_inff();
      lv[s] = s < mg.n ? ps[16 * HD + 16 + rl] : 0.0f;
      ov[s] = s < mg.n ? *reinterpret_cast<const f4*>(ps + rl * HD + c) : f4{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int s = 0; s < kMergeBatch; s++)
      if (s < mg.n) m = fmaxf(m, mv[s]);
#pragma unroll
    for (int s = 0; s < kMergeBatch; s++) {
      if (s >= mg.n || mv[s] == -__builtin_inff()) continue;
      const float w = __builtin_amdgcn_exp2f(mv[s] - m);
      l = l + lv[s] * w;
#pragma unroll
      for (int e = 0; e < 4; e++) o[e] = o[e] + ov[s][e] * w;
    }
  } else {
    for (int s = 0; s < mg.n; s++) m = fmaxf(m, p0[(int64_t)s * 32 * HD + 16 * HD + rl]);
    for (int s = 0; s < mg.n; s++) {
      const float* ps = p0 + (int64_t)s * 32 * HD;
      const float ms = ps[16 * HD + rl];
      if (ms == -__builtin_inff()) continue;
      const float w = __builtin_amdgcn_exp2f(ms - m);
      l = l + ps[16 * HD + 16 + rl] * w;
      const f4 os = *reinterpret_cast<const f4*>(ps + rl * HD + c);
#pragma unroll
      for (int e = 0; e < 4; e++) o[e] = o[e] + os[e] * w;
    }
  }
  f4 y;
#pragma unroll
  for (int e = 0; e < 4; e++) y[e] = __fdiv_rn(o[e], l);
  *reinterpret_cast<f4*>(a.o + ((int64_t)mg.rbase + row) * a.ldq + (int64_t)mg.head * HD + c) = y;
  if (c == 0) a.lse[(int64_t)mg.head * a.t + mg.rbase + row] = m * 0.693147180559945309417f + logf(l);
}

// ------------------------------------------------------------------ backward
// sums of a block's partials in slot order, one thread per four consecutive elements 4 e4 ..: dq
// (kv = false, 16 x hd) or dk then dv (kv = true, 2 x 16 x hd)
__device__ __forceinline__ void attn_merge_sum(const MAttnArgs& a, const MAttnMerge& mg, int e4, bool kv) {
  const int HD = a.hd, e = 4 * e4;
  const int part = e / (16 * HD), rl = (e % (16 * HD)) / HD, c = e % HD, row = mg.blk * 16 + rl;
  if (row >= a.t) return;
  const float* p0 = a.part + (int64_t)mg.s0 * (32 * HD) + e;
  f4 s = {0.0f, 0.0f, 0.0f, 0.0f};
  if (mg.n <= kMergeBatch) {  // loads together, summed in slot order
    f4 v[kMergeBatch];
#pragma unroll
    for (int k = 0; k < kMergeBatch; k++)
      v[k] = k < mg.n ? *reinterpret_cast<const f4*>(p0 + (int64_t)k * 32 * HD) : f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < kMergeBatch; k++)
      if (k < mg.n) s += v[k];
  } else {
    for (int k = 0; k < mg.n; k++) s += *reinterpret_cast<const f4*>(p0 + (int64_t)k * 32 * HD);
  }
  float* dst = !kv ? a.dq + (int64_t)row * a.ldq : part == 0 ? a.dk + (int64_t)row * a.ldk : a.dv + (int64_t)row * a.ld_dv;
  *reinterpret_cast<f4*>(dst + (int64_t)mg.head * HD + c) = s;
}

// merges: grid n_merges x ceil(elements / 1024) (flat), one thread per four elements of a block
#define RTQ_ATTN_MERGE_KERNEL(NAME, NEL, CALL)                                          \
  extern "C" __global__ __launch_bounds__(256) void NAME(MAttnArgs a) {                 \
    const int per = (NEL / 4 + 255) / 256, mi = blockIdx.x / per;                       \
    const int e4 = (blockIdx.x % per) * 256 + threadIdx.x;                              \
    if (mi < a.n_merges && e4 < NEL / 4) CALL;                                          \
  }
RTQ_ATTN_MERGE_KERNEL(rtq_m_attn_merge_fwd, 16 * a.hd, attn_merge_fwd(a, a.merges[mi], e4))
#undef RTQ_ATTN_MERGE_KERNEL
// the backward's merges in one launch: the dk / dv blocks (merges2, slots in part2; 32 x hd
// elements each) then the dq blocks (merges; 16 x hd)
extern "C" __global__ __launch_bounds__(256) void rtq_m_attn_merge_bwd(MAttnArgs a) {
  const int pk = (8 * a.hd + 255) / 256, pq = (4 * a.hd + 255) / 256;
  const int b = (int)blockIdx.x;
  if (b < a.n_merges2 * pk) {
    const int e4 = (b % pk) * 256 + threadIdx.x;
    MAttnArgs k = a;
    k.part = a.part2;
    if (e4 < 8 * a.hd) attn_merge_sum(k, a.merges2[b / pk], e4, true);
  } else {
    const int bq = b - a.n_merges2 * pk, mi = bq / pq, e4 = (bq % pq) * 256 + threadIdx.x;
    if (mi < a.n_merges && e4 < 4 * a.hd) attn_merge_sum(a, a.merges[mi], e4, false);
  }
}

// ------------------------------------------------------------------ packed forward: sequences
// gather: one workgroup per gathered row r of q (nh hd floats), k, v (nkv hd each) from packed row
// gmap[r] (rows with gmap[r] < 0 are zero), 16-byte loads and stores
extern "C" __global__ __launch_bounds__(256) void rtq_m_seq_gather(MSeqArgs a) {
  const int r = blockIdx.x;
  if (r >= a.tv) return;
  const int src = a.gmap[r];
  const int qd4 = a.nh * a.hd / 4, kd4 = a.nkv * a.hd / 4;
  const f4 z = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int e = threadIdx.x; e < qd4 + 2 * kd4; e += 256) {
    const float* s;
    float* d;
    if (e < qd4) {
      s = a.q + (int64_t)src * a.ldq + 4 * e;
      d = a.gq + (int64_t)r * (4 * qd4) + 4 * e;
    } else if (e < qd4 + kd4) {
      s = a.k + (int64_t)src * a.ldk + 4 * (e - qd4);
      d = a.gk + (int64_t)r * (4 * kd4) + 4 * (e - qd4);
    } else {
      s = a.v + (int64_t)src * a.ldv + 4 * (e - qd4 - kd4);
      d = a.gv + (int64_t)r * (4 * kd4) + 4 * (e - qd4 - kd4);
    }
    *reinterpret_cast<f4*>(d) = src >= 0 ? *reinterpret_cast<const f4*>(s) : z;
  }
}
// scatter: one workgroup per packed row i: o row from gathered row sidx[i] (and lse per head)
extern "C" __global__ __launch_bounds__(256) void rtq_m_seq_scatter(MSeqArgs a) {
  const int i = blockIdx.x;
  if (i >= a.t) return;
  const int src = a.sidx[i];
  const int qd4 = a.nh * a.hd / 4;
  for (int e = threadIdx.x; e < qd4; e += 256)
    *reinterpret_cast<f4*>(a.o + (int64_t)i * a.ldq + 4 * e) =
        *reinterpret_cast<const f4*>(a.go + (int64_t)src * (4 * qd4) + 4 * e);
  if (a.glse)
    for (int h = threadIdx.x; h < a.nh; h += 256) a.lse[(int64_t)h * a.t + i] = a.glse[(int64_t)h * a.tv + src];
}
