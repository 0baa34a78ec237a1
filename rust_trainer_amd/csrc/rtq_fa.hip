// rtq_fa.hip — fused causal GQA attention of the training step on 16-bit MFMA with LDS-shared
// tiles (Attention::forward / backward, src/attention.rs:187-235, :262-320); the probabilities are
// never stored.  Included by rtq_model_kernels.hip after rtq_attn.hip (whose masks, row helpers and
// merge kernels it shares).
//
// Work: a workgroup of four waves takes one item (MAttnItem) of 64 rows - 64 queries of one head
// (forward, dq) or 64 keys of one KV head (dk / dv) - wave w owning rows 16 w .. 16 w + 15, over
// the item's range of 64-wide tiles of the other side; each tile is staged in LDS once and shared
// by the four waves, the next tile's loads in registers while the current one is multiplied.
// Arithmetic, per product (acc is f32, the MFMA 16x16x32 output layout lane = column li, rows
// 4 g .. 4 g + 3):
//   forward S = (q scale) k^T, o = p v, and the backward's recomputed S: f16 MFMA; the stored k and
//     v are f16 values (kv_f16), staged exactly as one f16 plane; q scale and p are split into f16
//     hi = f16(x) and lo = f16(x - hi) (22 significant bits): acc += xh y + xl y;
//   backward dP = dO v^T, dq = dS k, dk = dS^T q, dv = p^T dO: bf16 MFMA, both operands split into
//     bf16 hi / lo, each rounded to nearest (f16 k and v split exactly), acc += xh yh + xl yh +
//     xh yl (a relative error near 2^-16 per product; bf16 keeps f32's exponent range, so gradients
//     below f16's range need no scaling).
// The scores are taken in base 2: q is scaled by scale log2(e), so p = 2^(s2 - m2) with the hardware
// exp2 (v_exp_f32); the stored lse stays natural (m2 ln 2 + log l) and the backward recomputes
// p = 2^(s2 - lse log2(e)).  Masks, online softmax (running max m2 and sum l per query row,
// rescaled by 2^(m_old - m_new)), D = dO . o, ds = (p (dp - D)) scale and the partial-slot merges
// follow rtq_attn.hip (whose forward merge reads base-2 maxima); the mask works on segments held
// in registers (the keys' per tile, the rows' per item).  An item covering part of its block's
// range writes its four 16-row sub-blocks to slots slot + w n (n = items of the block, in
// it.pad0), so each sub-block's partials are contiguous for rtq_m_attn_merge_*.

constexpr int kFaPad = 8;  // 16-bit elements of row padding: a lane group's 16 rows on distinct banks
constexpr float kLog2e = 1.44269504088896340736f, kLn2 = 0.693147180559945309417f;

// two floats -> packed f16 pair, rounded toward zero (one v_cvt_pkrtz; exact for f16 values)
__device__ __forceinline__ uint32_t fa_pk(float x, float y) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(x, y));
}
__device__ __forceinline__ float fa_lo16(uint32_t p) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(p & 0xffffu)); }
__device__ __forceinline__ float fa_hi16(uint32_t p) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(p >> 16)); }
// two floats -> f16 hi / lo pairs: hi = f16(x) toward zero, lo = f16(x - hi) (x - hi is exact in
// f32), 22 significant bits of x
__device__ __forceinline__ void fa_split_pair(float x, float y, uint32_t& hi, uint32_t& lo) {
  hi = fa_pk(x, y);
  lo = fa_pk(x - fa_lo16(hi), y - fa_hi16(hi));
}
__device__ __forceinline__ void fa_split_f16(const f4 v, u2v& hi, u2v& lo) {
  uint32_t h0, l0, h1, l1;
  fa_split_pair(v[0], v[1], h0, l0);
  fa_split_pair(v[2], v[3], h1, l1);
  hi = u2v{h0, h1};
  lo = u2v{l0, l1};
}
// four floats -> f16 (exact for f16 values), packed
__device__ __forceinline__ u2v fa_f16(const f4 v) { return u2v{fa_pk(v[0], v[1]), fa_pk(v[2], v[3])}; }
// one float -> bf16 hi / lo bits, each rounded to nearest even (v_cvt_pk_bf16_f32; x - hi is
// exact in f32): hi + lo holds x within 2^-17 of |x|
__device__ __forceinline__ void fa_split_bf(float x, uint32_t& hi, uint32_t& lo) {
  const __bf16 h = (__bf16)x;
  hi = __builtin_bit_cast(uint16_t, h);
  lo = __builtin_bit_cast(uint16_t, (__bf16)(x - (float)h));
}
__device__ __forceinline__ half8 fa_h8(const uint16_t* p) { return *reinterpret_cast<const half8*>(p); }
__device__ __forceinline__ bf8 fa_b8(const uint16_t* p) { return *reinterpret_cast<const bf8*>(p); }

// ---- tile staging: 64 rows x HD of X (rows r0 + i, stride ld, clamped to t - 1), 256 threads
// natural layout [row][d]: thread -> row tid / 4, columns (tid % 4) HD / 4 .. (NF float4)
template <int HD>
struct FaNat {
  static constexpr int NF = HD / 16;
  f4 v[NF];
  __device__ __forceinline__ void load(const float* X, int64_t ld, int r0, int t) {
    const float* p = X + (int64_t)min(r0 + (int)(threadIdx.x >> 2), t - 1) * ld + (threadIdx.x & 3) * (HD / 4);
#pragma unroll
    for (int i = 0; i < NF; i++) v[i] = *reinterpret_cast<const f4*>(p + 4 * i);
  }
};
// transposed layout [d][row]: thread -> rows KPT kg .. (kg = tid / (HD / 4)), columns 4 (tid % (HD / 4)) ..
template <int HD>
struct FaTr {
  static constexpr int KPT = HD / 16;  // rows per thread: 8 (HD 128) or 4 (HD 64)
  f4 v[KPT];
  __device__ __forceinline__ void load(const float* X, int64_t ld, int r0, int t) {
    const int kg = threadIdx.x / (HD / 4), d4 = threadIdx.x % (HD / 4);
#pragma unroll
    for (int i = 0; i < KPT; i++)
      v[i] = *reinterpret_cast<const f4*>(X + (int64_t)min(r0 + kg * KPT + i, t - 1) * ld + 4 * d4);
  }
};
// stores: f16 one plane (exact values), natural
template <int HD, int LD>
__device__ __forceinline__ void fa_store_nat_f16(const FaNat<HD>& s, uint16_t* P) {
  uint16_t* p = P + (threadIdx.x >> 2) * LD + (threadIdx.x & 3) * (HD / 4);
#pragma unroll
  for (int i = 0; i < FaNat<HD>::NF; i++) *reinterpret_cast<u2v*>(p + 4 * i) = fa_f16(s.v[i]);
}
// transposed store [d][row] (row stride LD): f16 one plane
template <int HD, int LD>
__device__ __forceinline__ void fa_store_tr_f16(const FaTr<HD>& s, uint16_t* P) {
  constexpr int KPT = FaTr<HD>::KPT;
  const int kg = threadIdx.x / (HD / 4), d4 = threadIdx.x % (HD / 4);
#pragma unroll
  for (int c = 0; c < 4; c++) {
    uint16_t* p = P + (4 * d4 + c) * LD + kg * KPT;
    if constexpr (KPT == 8)
      *reinterpret_cast<u4v*>(p) = u4v{fa_pk(s.v[0][c], s.v[1][c]), fa_pk(s.v[2][c], s.v[3][c]),
                                       fa_pk(s.v[4][c], s.v[5][c]), fa_pk(s.v[6][c], s.v[7][c])};
    else
      *reinterpret_cast<u2v*>(p) = u2v{fa_pk(s.v[0][c], s.v[1][c]), fa_pk(s.v[2][c], s.v[3][c])};
  }
}
// a 16 x 64 tile in MFMA output order (tv[j][i]: row 4 g + i, column 16 j + li) -> two 16-bit planes
// [row][col] (stride 64 + kFaPad) of the wave: f16 hi / lo (HF) or bf16 hi / lo
template <bool HF>
__device__ __forceinline__ void fa_put_tile(const float (&tv)[4][4], uint16_t* Th, uint16_t* Tl) {
  constexpr int LD = 64 + kFaPad;
  const int lane = threadIdx.x & 63, li = lane & 15, g = lane >> 4;
#pragma unroll
  for (int i = 0; i < 4; i += 2)
#pragma unroll
    for (int j = 0; j < 4; j++) {
      uint32_t h, l;  // rows 4 g + i (low halves) and 4 g + i + 1 (high halves)
      if (HF) {
        fa_split_pair(tv[j][i], tv[j][i + 1], h, l);
      } else {
        uint32_t h0, l0, h1, l1;
        fa_split_bf(tv[j][i], h0, l0);
        fa_split_bf(tv[j][i + 1], h1, l1);
        h = h0 | (h1 << 16);
        l = l0 | (l1 << 16);
      }
      Th[(4 * g + i) * LD + 16 * j + li] = (uint16_t)(h & 0xffffu);
      Tl[(4 * g + i) * LD + 16 * j + li] = (uint16_t)(l & 0xffffu);
      Th[(4 * g + i + 1) * LD + 16 * j + li] = (uint16_t)(h >> 16);
      Tl[(4 * g + i + 1) * LD + 16 * j + li] = (uint16_t)(l >> 16);
    }
}

// may query i (segment si) attend to key j (segment sj)?  (attn_ok with both segments in registers:
// no load under the condition)
__device__ __forceinline__ bool fa_ok(int i, int j, int si, int sj, int t) { return j <= i && i < t && (sj == 0 || sj == si); }

// the next live 64-wide tile of rows r0 (64-block qb) at or after kt, below b1
__device__ __forceinline__ int fa_next_live(const MAttnArgs& a, int qb, int kt, int b1) {
  while (kt < b1 && !attn_tile_live(a, qb, kt)) kt++;
  return kt;
}

// ------------------------------------------------------------------ forward
template <int HD>
struct FaFwdLds {
  static constexpr int LDK = HD + kFaPad, LDV = 64 + kFaPad;
  uint16_t k[64 * LDK];    // K tile [key][d], f16
  uint16_t vt[HD * LDV];   // V tile [d][key], f16
  uint16_t ph[4][16 * LDV], pl[4][16 * LDV];  // per wave: p [row][key], f16 hi / lo
};

template <int HD>
__device__ __forceinline__ void fa_fwd(const MAttnArgs& a, const MAttnItem& it, FaFwdLds<HD>& L) {
  constexpr int NC = HD / 16, NK = HD / 32, LDK = FaFwdLds<HD>::LDK, LDV = FaFwdLds<HD>::LDV;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, li = lane & 15, g = lane >> 4;
  const int h = it.head, kvh = h / (a.nh / a.nkv), qb = it.blk, r0 = qb * 64 + 16 * w;
  // the item's sequence: rows [rbase, rbase + tl) (the whole step, or a packed layout's segment
  // gathered; the mask and the clamps work on its rows)
  const int tl = it.rlen;
  const int64_t rb = it.rbase;
  // q rows of the wave times scale log2(e) (scores in base 2: p = 2^(s2 - m2)), f16 hi / lo
  // operand fragments
  const float qs2 = a.scale * kLog2e;
  half8 qh[NK], ql[NK];
  {
    const float* qr = a.q + (rb + min(r0 + li, tl - 1)) * a.ldq + (int64_t)h * HD + 8 * g;
#pragma unroll
    for (int c = 0; c < NK; c++) {
      u2v h0, l0, h1, l1;
      fa_split_f16(*reinterpret_cast<const f4*>(qr + 32 * c) * qs2, h0, l0);
      fa_split_f16(*reinterpret_cast<const f4*>(qr + 32 * c + 4) * qs2, h1, l1);
      qh[c] = __builtin_bit_cast(half8, u4v{h0.x, h0.y, h1.x, h1.y});
      ql[c] = __builtin_bit_cast(half8, u4v{l0.x, l0.y, l1.x, l1.y});
    }
  }
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
  const float* kb = a.k + rb * a.ldk + (int64_t)kvh * HD;
  const float* vb = a.v + rb * a.ldv + (int64_t)kvh * HD;
  FaNat<HD> kn;
  FaTr<HD> vn;
  int kt = fa_next_live(a, qb, it.b0, it.b1);
  if (kt < it.b1) {
    kn.load(kb, a.ldk, kt * 64, tl);
    vn.load(vb, a.ldv, kt * 64, tl);
  }
  while (kt < it.b1) {  // kt is workgroup-uniform: every wave runs the same barriers
    const int k0 = kt * 64;
    fa_store_nat_f16<HD, LDK>(kn, L.k);
    fa_store_tr_f16<HD, LDV>(vn, L.vt);
    __syncthreads();
    const int kt2 = fa_next_live(a, qb, kt + 1, it.b1);
    if (kt2 < it.b1) {
      kn.load(kb, a.ldk, kt2 * 64, tl);
      vn.load(vb, a.ldv, kt2 * 64, tl);
    }
    f4 s[4] = {zero, zero, zero, zero};
#pragma unroll
    for (int c = 0; c < NK; c++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const half8 kf = fa_h8(L.k + (16 * j + li) * LDK + 32 * c + 8 * g);
        s[j] = mfma_f16(qh[c], kf, s[j]);
        s[j] = mfma_f16(ql[c], kf, s[j]);
      }
    float p[4][4];
    int sk[4];  // segments of the lane's keys
#pragma unroll
    for (int j = 0; j < 4; j++) sk[j] = attn_seg(a, k0 + 16 * j + li);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int row = r0 + 4 * g + i;
      float mx = -__builtin_inff();
#pragma unroll
      for (int j = 0; j < 4; j++) {
        p[j][i] = fa_ok(row, k0 + 16 * j + li, si[i], sk[j], tl) ? s[j][i] : -__builtin_inff();
        mx = fmaxf(mx, p[j][i]);
      }
      mx = group16_max(mx);
      const float mn = fmaxf(mr[i], mx);
      const bool none = mn == -__builtin_inff();  // no key of the row so far
      const float corr = mr[i] == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(mr[i] - mn);
      float ls = 0.0f;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        p[j][i] = none ? 0.0f : __builtin_amdgcn_exp2f(p[j][i] - mn);  // 2^-inf = 0 for masked keys
        ls = ls + p[j][i];
      }
      ls = group16_sum(ls);
      lr[i] = lr[i] * corr + ls;
      mr[i] = mn;
#pragma unroll
      for (int c = 0; c < NC; c++) oacc[c][i] = oacc[c][i] * corr;
    }
    fa_put_tile<true>(p, L.ph[w], L.pl[w]);
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int c = 0; c < 2; c++) {
      const half8 ph = fa_h8(L.ph[w] + li * LDV + 32 * c + 8 * g);
      const half8 pl = fa_h8(L.pl[w] + li * LDV + 32 * c + 8 * g);
#pragma unroll
      for (int cc = 0; cc < NC; cc++) {
        const half8 vf = fa_h8(L.vt + (16 * cc + li) * LDV + 32 * c + 8 * g);
        oacc[cc] = mfma_f16(ph, vf, oacc[cc]);
        oacc[cc] = mfma_f16(pl, vf, oacc[cc]);
      }
    }
    __syncthreads();  // every wave is done with this tile's K, V (and its own p) before the next store
    kt = kt2;
  }
  if (it.slot < 0) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int row = r0 + 4 * g + i;
      if (row >= tl) continue;
      float* orow = a.o + (rb + row) * a.ldq + (int64_t)h * HD + li;
#pragma unroll
      for (int c = 0; c < NC; c++) orow[16 * c] = __fdiv_rn(oacc[c][i], lr[i]);
      if (li == 0) a.lse[(int64_t)h * a.t + rb + row] = mr[i] * kLn2 + logf(lr[i]);  // natural log-sum-exp
    }
  } else {  // partials: o, m (base 2), l
    float* pp = a.part + (int64_t)(it.slot + w * it.pad0) * (32 * HD);
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

// ------------------------------------------------------------------ backward operand planes
// One workgroup per (16-token group, head) of q / dO / o (heads [0, nh)) or of k / v (kv heads
// after them), 256 threads, in two independent parts (no barrier):
//   natural planes and D = dO . o: thread -> token tid / 16 of the group, columns (tid % 16) HD / 16
//     .. (rows past t not written: the readers clamp rows to t - 1);
//   transposed planes: thread -> column d = tid / (256 / HD), tokens TPT (tid % (256 / HD)) .. of
//     the group (TPT = HD / 16), read down the column (each load instruction of a wave covers whole
//     row segments) and written as one TPT-half piece per plane (tokens past t zero).
template <int HD>
__device__ __forceinline__ void fa_bwd_prep(const MAttnArgs& a) {
  constexpr int NC = HD / 16, TPT = HD / 16, TPD = 256 / HD;  // columns per thread; tokens per thread
  const int tg = blockIdx.x, hb = blockIdx.y, tid = threadIdx.x;
  const bool kvs = hb >= a.nh;
  const int h = kvs ? hb - a.nh : hb, heads = kvs ? a.nkv : a.nh;
  // the transposed planes' values (column d, tokens t0 .. t0 + TPT - 1) are loaded first, so that
  // their round trip overlaps the natural planes' (stores to the planes could alias the sources)
  const int d = tid / TPD, t0 = tg * 16 + (tid % TPD) * TPT;
  auto col_ld = [&](const float* X, int64_t ldx, float (&v)[TPT]) {
#pragma unroll
    for (int j = 0; j < TPT; j++) v[j] = t0 + j < a.t ? X[(int64_t)(t0 + j) * ldx + (int64_t)h * HD + d] : 0.0f;
  };
  float c1[TPT], c2[TPT];
  if (!kvs) {
    col_ld(a.q, a.ldq, c1);
    col_ld(a.dO, a.ldq, c2);
  } else {
    col_ld(a.k, a.ldk, c1);
  }
  {  // natural planes (+ D)
    const int t = tg * 16 + (tid >> 4), c0 = (tid & 15) * NC;
    const bool in = t < a.t;
    const int tc = min(t, a.t - 1);
    const int64_t no = ((int64_t)t * heads + h) * HD + c0;
    auto ld = [&](const float* X, int64_t ldx, float (&v)[NC]) {
      const float* p = X + (int64_t)tc * ldx + (int64_t)h * HD + c0;
#pragma unroll
      for (int i = 0; i < NC; i += 4) {
        const f4 q = *reinterpret_cast<const f4*>(p + i);
        v[i] = q.x, v[i + 1] = q.y, v[i + 2] = q.z, v[i + 3] = q.w;
      }
    };
    auto put_bf = [&](const float (&v)[NC], uint16_t* Ph, uint16_t* Pl) {
#pragma unroll
      for (int i = 0; i < NC; i += 4) {
        uint32_t bh[4], bl[4];
#pragma unroll
        for (int e = 0; e < 4; e++) fa_split_bf(v[i + e], bh[e], bl[e]);
        *reinterpret_cast<u2v*>(Ph + no + i) = u2v{bh[0] | (bh[1] << 16), bh[2] | (bh[3] << 16)};
        *reinterpret_cast<u2v*>(Pl + no + i) = u2v{bl[0] | (bl[1] << 16), bl[2] | (bl[3] << 16)};
      }
    };
    if (!kvs) {
      float qv[NC], dv[NC], ov[NC];
      ld(a.q, a.ldq, qv);
      ld(a.dO, a.ldq, dv);
      ld(a.o, a.ldq, ov);
      float s = 0.0f;  // D: the thread's columns in order, then the token's 16 lanes (fixed order)
#pragma unroll
      for (int i = 0; i < NC; i++) s = s + dv[i] * ov[i];
#pragma unroll
      for (int m = 1; m < 16; m <<= 1) s = s + __shfl_xor(s, m);
      if (in) {
        if ((tid & 15) == 0) a.D[(int64_t)h * a.t + t] = s;
        const float qs2 = a.scale * kLog2e;  // scores in base 2
#pragma unroll
        for (int i = 0; i < NC; i += 4) {
          u2v hi, lo;
          fa_split_f16(f4{qv[i], qv[i + 1], qv[i + 2], qv[i + 3]} * qs2, hi, lo);
          *reinterpret_cast<u2v*>(a.pqsh + no + i) = hi;
          *reinterpret_cast<u2v*>(a.pqsl + no + i) = lo;
        }
        put_bf(dv, a.pdoh, a.pdol);
      }
    } else {
      float kv[NC], vv[NC];
      ld(a.k, a.ldk, kv);
      ld(a.v, a.ldv, vv);
      if (in) {
#pragma unroll
        for (int i = 0; i < NC; i += 4) *reinterpret_cast<u2v*>(a.pkf + no + i) = fa_f16(f4{kv[i], kv[i + 1], kv[i + 2], kv[i + 3]});
        put_bf(vv, a.pvh, a.pvl);
      }
    }
  }
  {  // transposed planes: column d, tokens t0 .. t0 + TPT - 1
    auto col = [&](const float (&v)[TPT], uint16_t* Ph, uint16_t* Pl) {
      uint32_t bh[TPT], bl[TPT];
#pragma unroll
      for (int j = 0; j < TPT; j++) fa_split_bf(v[j], bh[j], bl[j]);
      const int64_t go = ((int64_t)h * HD + d) * a.tp + t0;
      if constexpr (TPT == 8) {
        *reinterpret_cast<u4v*>(Ph + go) = u4v{bh[0] | (bh[1] << 16), bh[2] | (bh[3] << 16), bh[4] | (bh[5] << 16), bh[6] | (bh[7] << 16)};
        *reinterpret_cast<u4v*>(Pl + go) = u4v{bl[0] | (bl[1] << 16), bl[2] | (bl[3] << 16), bl[4] | (bl[5] << 16), bl[6] | (bl[7] << 16)};
      } else {
        *reinterpret_cast<u2v*>(Ph + go) = u2v{bh[0] | (bh[1] << 16), bh[2] | (bh[3] << 16)};
        *reinterpret_cast<u2v*>(Pl + go) = u2v{bl[0] | (bl[1] << 16), bl[2] | (bl[3] << 16)};
      }
    };
    if (!kvs) {
      col(c1, a.pqth, a.pqtl);
      col(c2, a.pdth, a.pdtl);
    } else {
      col(c1, a.pkth, a.pktl);
    }
  }
}
extern "C" __global__ __launch_bounds__(256) void rtq_m_attn_bwd_prep64(MAttnArgs a) { fa_bwd_prep<64>(a); }
extern "C" __global__ __launch_bounds__(256) void rtq_m_attn_bwd_prep128(MAttnArgs a) { fa_bwd_prep<128>(a); }

// 16-byte copies of plane rows into LDS: n16 pieces of a row-major [rows][rowlen] source (row
// stride ld halves, rows clamped to rmax) -> [rows][LD] in LDS, rowlen a multiple of 8 halves
template <int ROWS, int ROWLEN, int LD>
struct FaCopy {
  static constexpr int PIECES = ROWS * ROWLEN / 8, PER = (PIECES + 255) / 256;
  u4v v[PER];
  __device__ __forceinline__ void load(const uint16_t* P, int64_t ld, int r0, int rmax) {
#pragma unroll
    for (int k = 0; k < PER; k++) {
      const int u = threadIdx.x + 256 * k, row = u / (ROWLEN / 8), p8 = u % (ROWLEN / 8);
      if (PIECES % 256 == 0 || u < PIECES)
        v[k] = *reinterpret_cast<const u4v*>(P + (int64_t)min(r0 + row, rmax) * ld + 8 * p8);
    }
  }
  __device__ __forceinline__ void store(uint16_t* L) const {
#pragma unroll
    for (int k = 0; k < PER; k++) {
      const int u = threadIdx.x + 256 * k, row = u / (ROWLEN / 8), p8 = u % (ROWLEN / 8);
      if (PIECES % 256 == 0 || u < PIECES) *reinterpret_cast<u4v*>(L + row * LD + 8 * p8) = v[k];
    }
  }
};

// ------------------------------------------------------------------ dq
// Item: 64 queries (it.blk) of head it.head over the 64-key tiles [b0, b1).  Wave w = (wq, wh) =
// (w / 2, w % 2) owns queries 32 wq .. 32 wq + 31 (two 16-row tiles, their q scale and dO operand
// fragments in registers); it forms S and dP for the key half 32 wh .. 32 wh + 31 of each tile and
// dq for the column half (HD / 2) wh .. of its queries, so every K / V fragment read from LDS feeds
// both row tiles.  dS of the whole 64 x 64 tile passes between the two phases through LDS.
template <int HD>
struct FaDqLds {
  static constexpr int LDK = HD + kFaPad, LDT = 64 + kFaPad;
  uint16_t k[64 * LDK];                  // K [key][d], f16 (S)
  uint16_t vh[64 * LDK], vl[64 * LDK];   // V [key][d], bf16 hi / lo (dP = dO V^T)
  uint16_t kth[HD * LDT], ktl[HD * LDT]; // K [d][key], bf16 hi / lo (dq = dS K)
  uint16_t sh[64 * LDT], sl[64 * LDT];   // dS [query][key], bf16 hi / lo
};

template <int HD>
__device__ __forceinline__ void fa_dq(const MAttnArgs& a, const MAttnItem& it, FaDqLds<HD>& L) {
  constexpr int NC = HD / 16, NH = NC / 2, NK = HD / 32, LDK = FaDqLds<HD>::LDK, LDT = FaDqLds<HD>::LDT;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, li = lane & 15, g = lane >> 4;
  const int wq = w >> 1, wh = w & 1;
  const int h = it.head, kvh = h / (a.nh / a.nkv), qb = it.blk, r0 = qb * 64 + 32 * wq;
  half8 qh[2][NK], ql[2][NK];  // q scale log2(e) (f16 hi / lo) and dO (bf16 hi / lo) from the planes
  bf8 dh[2][NK], dl[2][NK];
#pragma unroll
  for (int u = 0; u < 2; u++) {
    const int64_t o = ((int64_t)min(r0 + 16 * u + li, a.t - 1) * a.nh + h) * HD + 8 * g;
#pragma unroll
    for (int c = 0; c < NK; c++) {
      qh[u][c] = fa_h8(a.pqsh + o + 32 * c);
      ql[u][c] = fa_h8(a.pqsl + o + 32 * c);
      dh[u][c] = fa_b8(a.pdoh + o + 32 * c);
      dl[u][c] = fa_b8(a.pdol + o + 32 * c);
    }
  }
  int si[2][4];
  float lq[2][4], Dq[2][4];
#pragma unroll
  for (int u = 0; u < 2; u++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int row = min(r0 + 16 * u + 4 * g + i, a.t - 1);
      si[u][i] = attn_seg(a, row);
      lq[u][i] = a.lse[(int64_t)h * a.t + row] * kLog2e;
      Dq[u][i] = a.D[(int64_t)h * a.t + row];
    }
  const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  f4 acc[2][NH];  // [query tile][column tile NH wh + cc]
#pragma unroll
  for (int u = 0; u < 2; u++)
#pragma unroll
    for (int c = 0; c < NH; c++) acc[u][c] = zero;
  // staging: plain copies of the planes (K f16, V bf16 hi / lo natural; K bf16 hi / lo transposed)
  const int64_t kvo = (int64_t)kvh * HD, ldn = (int64_t)a.nkv * HD;
  FaCopy<64, HD, LDK> ck, cvh, cvl;
  FaCopy<HD, 64, LDT> ckh, ckl;
  auto load_tile = [&](int ktile) {
    const int k0 = ktile * 64;
    ck.load(a.pkf + kvo, ldn, k0, a.t - 1);
    cvh.load(a.pvh + kvo, ldn, k0, a.t - 1);
    cvl.load(a.pvl + kvo, ldn, k0, a.t - 1);
    ckh.load(a.pkth + k0, a.tp, (int)kvo, 1 << 30);
    ckl.load(a.pktl + k0, a.tp, (int)kvo, 1 << 30);
  };
  int kt = fa_next_live(a, qb, it.b0, it.b1);
  if (kt < it.b1) load_tile(kt);
  while (kt < it.b1) {
    const int k0 = kt * 64;
    ck.store(L.k);
    cvh.store(L.vh);
    cvl.store(L.vl);
    ckh.store(L.kth);
    ckl.store(L.ktl);
    __syncthreads();
    const int kt2 = fa_next_live(a, qb, kt + 1, it.b1);
    if (kt2 < it.b1) load_tile(kt2);
    // S and dP of the two query tiles x keys 32 wh + 16 j (j = 0, 1)
    f4 s[2][2] = {{zero, zero}, {zero, zero}}, dp[2][2] = {{zero, zero}, {zero, zero}};
#pragma unroll
    for (int c = 0; c < NK; c++)
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const int o = (32 * wh + 16 * j + li) * LDK + 32 * c + 8 * g;
        const half8 kf = fa_h8(L.k + o);
        const bf8 vh = fa_b8(L.vh + o), vl = fa_b8(L.vl + o);
#pragma unroll
        for (int u = 0; u < 2; u++) {
          s[u][j] = mfma_f16(qh[u][c], kf, s[u][j]);
          s[u][j] = mfma_f16(ql[u][c], kf, s[u][j]);
          dp[u][j] = mfma_bf16(dh[u][c], vh, dp[u][j]);
          dp[u][j] = mfma_bf16(dl[u][c], vh, dp[u][j]);
          dp[u][j] = mfma_bf16(dh[u][c], vl, dp[u][j]);
        }
      }
    int sk[2];
#pragma unroll
    for (int j = 0; j < 2; j++) sk[j] = attn_seg(a, k0 + 32 * wh + 16 * j + li);
    // dS -> LDS [query 32 wq + 16 u + 4 g + i][key 32 wh + 16 j + li], bf16 hi / lo
#pragma unroll
    for (int u = 0; u < 2; u++)
#pragma unroll
      for (int j = 0; j < 2; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int qrow = r0 + 16 * u + 4 * g + i, key = k0 + 32 * wh + 16 * j + li;
          const bool ok = fa_ok(qrow, key, si[u][i], sk[j], a.t);
          const float p = __builtin_amdgcn_exp2f(s[u][j][i] - lq[u][i]);
          const float ds = ok ? (p * (dp[u][j][i] - Dq[u][i])) * a.scale : 0.0f;
          uint32_t hb, lb;
          fa_split_bf(ds, hb, lb);
          const int o = (32 * wq + 16 * u + 4 * g + i) * LDT + 32 * wh + 16 * j + li;
          L.sh[o] = (uint16_t)hb;
          L.sl[o] = (uint16_t)lb;
        }
    __syncthreads();
    // dq[query tile u][column tile NH wh + cc] += dS K over the tile's 64 keys (two 32-key steps)
#pragma unroll
    for (int c = 0; c < 2; c++) {
      bf8 sh[2], sl[2];
#pragma unroll
      for (int u = 0; u < 2; u++) {
        sh[u] = fa_b8(L.sh + (32 * wq + 16 * u + li) * LDT + 32 * c + 8 * g);
        sl[u] = fa_b8(L.sl + (32 * wq + 16 * u + li) * LDT + 32 * c + 8 * g);
      }
#pragma unroll
      for (int cc = 0; cc < NH; cc++) {
        const int o = (16 * (NH * wh + cc) + li) * LDT + 32 * c + 8 * g;
        const bf8 kh = fa_b8(L.kth + o), kl = fa_b8(L.ktl + o);
#pragma unroll
        for (int u = 0; u < 2; u++) {
          acc[u][cc] = mfma_bf16(sh[u], kh, acc[u][cc]);
          acc[u][cc] = mfma_bf16(sl[u], kh, acc[u][cc]);
          acc[u][cc] = mfma_bf16(sh[u], kl, acc[u][cc]);
        }
      }
    }
    __syncthreads();
    kt = kt2;
  }
  if (it.slot < 0) {
#pragma unroll
    for (int u = 0; u < 2; u++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int row = r0 + 16 * u + 4 * g + i;
        if (row >= a.t) continue;
        float* q = a.dq + (int64_t)row * a.ldq + (int64_t)h * HD + 16 * NH * wh + li;
#pragma unroll
        for (int c = 0; c < NH; c++) q[16 * c] = acc[u][c][i];
      }
  } else {  // 16-row sub-block 2 wq + u of the item -> its slot; this wave's column half
#pragma unroll
    for (int u = 0; u < 2; u++) {
      float* pp = a.part + (int64_t)(it.slot + (2 * wq + u) * it.pad0) * (32 * HD) + 16 * NH * wh + li;
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int c = 0; c < NH; c++) pp[(4 * g + i) * HD + 16 * c] = acc[u][c][i];
    }
  }
}

// ------------------------------------------------------------------ dk, dv
// Item: 64 keys (it.blk) of KV head it.head over (group head, 64-query tile) pairs [b0, b1); each
// pair is taken as two 32-query halves (steps), staged as q scale (f16 hi / lo, [q][d], for S^T =
// k q^T), q (bf16 hi / lo, [d][q], for dk += dS^T q), dO (bf16 hi / lo, [q][d] for dP^T = v dO^T
// and [d][q] for dv += p^T dO).  Wave w = (wk, wh) = (w / 2, w % 2) owns keys 32 wk .. 32 wk + 31
// (two 16-key tiles, their k / v operand fragments in registers); it forms S^T and dP^T for the
// query half 16 wh .. 16 wh + 15 of the step and dk / dv for the column half (HD / 2) wh .. of its
// keys, so every q / dO fragment read from LDS feeds both key tiles.  p^T and dS^T of the whole
// 64 x 32 step pass between the two phases through LDS.
template <int HD>
struct FaKvLds {
  static constexpr int LDN = HD + kFaPad, LDT = 32 + kFaPad, LDP = 32 + kFaPad;
  uint16_t qsh[32 * LDN], qsl[32 * LDN];    // q scale [q][d], f16 hi / lo
  uint16_t qth[HD * LDT], qtl[HD * LDT];    // q [d][q], bf16 hi / lo
  uint16_t dsh_[32 * LDN], dsl_[32 * LDN];  // dO [q][d], bf16 hi / lo
  uint16_t dth[HD * LDT], dtl[HD * LDT];    // dO [d][q], bf16 hi / lo
  uint16_t ph[64 * LDP], pl[64 * LDP], sh[64 * LDP], sl[64 * LDP];  // p^T, dS^T [key][q], bf16 hi / lo
};
template <int HD>
__device__ __forceinline__ void fa_dkv(const MAttnArgs& a, const MAttnItem& it, FaKvLds<HD>& L) {
  constexpr int NC = HD / 16, NH = NC / 2, NK = HD / 32;
  constexpr int LDN = FaKvLds<HD>::LDN, LDT = FaKvLds<HD>::LDT, LDP = FaKvLds<HD>::LDP;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, li = lane & 15, g = lane >> 4;
  const int wk = w >> 1, wh = w & 1;
  const int kvh = it.head, grp = a.nh / a.nkv, kbk = it.blk, c0 = kbk * 64 + 32 * wk, nqt = (a.t + 63) / 64;
  // the wave's 32 keys: k (f16, exact) and v (bf16 hi / lo) operand fragments of its two key tiles
  half8 kf[2][NK];  // k (f16) and v (bf16 hi / lo) from the planes
  bf8 vh[2][NK], vl[2][NK];
#pragma unroll
  for (int u = 0; u < 2; u++) {
    const int64_t o = ((int64_t)min(c0 + 16 * u + li, a.t - 1) * a.nkv + kvh) * HD + 8 * g;
#pragma unroll
    for (int c = 0; c < NK; c++) {
      kf[u][c] = fa_h8(a.pkf + o + 32 * c);
      vh[u][c] = fa_b8(a.pvh + o + 32 * c);
      vl[u][c] = fa_b8(a.pvl + o + 32 * c);
    }
  }
  int skey[2][4];  // segments of the lane's keys c0 + 16 u + 4 g + i
#pragma unroll
  for (int u = 0; u < 2; u++)
#pragma unroll
    for (int i = 0; i < 4; i++) skey[u][i] = attn_seg(a, c0 + 16 * u + 4 * g + i);
  const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  f4 dk[2][NH], dv[2][NH];  // [key tile][column tile NH wh + cc]
#pragma unroll
  for (int u = 0; u < 2; u++)
#pragma unroll
    for (int c = 0; c < NH; c++) dk[u][c] = dv[u][c] = zero;
  // (pair, half) steps: pair pr = (group head, 64-query tile), half hf = 32-query half
  auto live_pair = [&](int pr) {
    const int qt = pr % nqt;
    return qt * 64 + 63 >= kbk * 64 && attn_tile_live(a, qt, kbk);
  };
  auto next_step = [&](int st) {  // step st = 2 pr + hf; the next live one at or after st
    while (st < 2 * it.b1 && !live_pair(st >> 1)) st = ((st >> 1) + 1) * 2;
    return st;
  };
  // staging: plain copies of the planes (q scale f16 and dO bf16 hi / lo natural; q, dO bf16 hi /
  // lo transposed)
  FaCopy<32, HD, LDN> cqh, cql, cdh, cdl;
  FaCopy<HD, 32, LDT> cqth, cqtl, cdth, cdtl;
  const int64_t ldn = (int64_t)a.nh * HD;
  auto load_step = [&](int st) {
    const int pr = st >> 1, h = kvh * grp + pr / nqt, q0 = (pr % nqt) * 64 + 32 * (st & 1);
    const int64_t ho = (int64_t)h * HD;
    cqh.load(a.pqsh + ho, ldn, q0, a.t - 1);
    cql.load(a.pqsl + ho, ldn, q0, a.t - 1);
    cdh.load(a.pdoh + ho, ldn, q0, a.t - 1);
    cdl.load(a.pdol + ho, ldn, q0, a.t - 1);
    cqth.load(a.pqth + q0, a.tp, (int)ho, 1 << 30);
    cqtl.load(a.pqtl + q0, a.tp, (int)ho, 1 << 30);
    cdth.load(a.pdth + q0, a.tp, (int)ho, 1 << 30);
    cdtl.load(a.pdtl + q0, a.tp, (int)ho, 1 << 30);
  };
  int st = next_step(2 * it.b0);
  if (st < 2 * it.b1) load_step(st);
  while (st < 2 * it.b1) {  // workgroup-uniform
    const int pr = st >> 1, h = kvh * grp + pr / nqt, q0 = (pr % nqt) * 64 + 32 * (st & 1);
    cqh.store(L.qsh);  // q scale log2(e): scores in base 2
    cql.store(L.qsl);
    cdh.store(L.dsh_);
    cdl.store(L.dsl_);
    cqth.store(L.qth);
    cqtl.store(L.qtl);
    cdth.store(L.dth);
    cdtl.store(L.dtl);
    __syncthreads();
    const int st2 = next_step(st + 1);
    if (st2 < 2 * it.b1) load_step(st2);
    // S^T = k (q scale)^T and dP^T = v dO^T: the two key tiles x queries 16 wh .. 16 wh + 15
    f4 s[2] = {zero, zero}, dp[2] = {zero, zero};
#pragma unroll
    for (int c = 0; c < NK; c++) {
      const int o = (16 * wh + li) * LDN + 32 * c + 8 * g;
      const half8 qhf = fa_h8(L.qsh + o), qlf = fa_h8(L.qsl + o);
      const bf8 dhf = fa_b8(L.dsh_ + o), dlf = fa_b8(L.dsl_ + o);
#pragma unroll
      for (int u = 0; u < 2; u++) {
        s[u] = mfma_f16(kf[u][c], qhf, s[u]);
        s[u] = mfma_f16(kf[u][c], qlf, s[u]);
        dp[u] = mfma_bf16(vh[u][c], dhf, dp[u]);
        dp[u] = mfma_bf16(vl[u][c], dhf, dp[u]);
        dp[u] = mfma_bf16(vh[u][c], dlf, dp[u]);
      }
    }
    {  // p^T, dS^T -> LDS [key 32 wk + 16 u + 4 g + i][query 16 wh + li], bf16 hi / lo
      const int qr = q0 + 16 * wh + li, qc = min(qr, a.t - 1);
      const float lq = a.lse[(int64_t)h * a.t + qc] * kLog2e, Dq = a.D[(int64_t)h * a.t + qc];
      const int sq = attn_seg(a, qc);
#pragma unroll
      for (int u = 0; u < 2; u++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const bool ok = fa_ok(qr, c0 + 16 * u + 4 * g + i, sq, skey[u][i], a.t);
          const float p = ok ? __builtin_amdgcn_exp2f(s[u][i] - lq) : 0.0f;
          const float ds = ok ? (p * (dp[u][i] - Dq)) * a.scale : 0.0f;
          uint32_t h0, l0, h1, l1;
          fa_split_bf(p, h0, l0);
          fa_split_bf(ds, h1, l1);
          const int o = (32 * wk + 16 * u + 4 * g + i) * LDP + 16 * wh + li;
          L.ph[o] = (uint16_t)h0;
          L.pl[o] = (uint16_t)l0;
          L.sh[o] = (uint16_t)h1;
          L.sl[o] = (uint16_t)l1;
        }
    }
    __syncthreads();
    {  // dV += P^T dO, dK += dS^T q over the step's 32 queries (one 32-deep MFMA step)
      bf8 phf[2], plf[2], shf[2], slf[2];
#pragma unroll
      for (int u = 0; u < 2; u++) {
        const int o = (32 * wk + 16 * u + li) * LDP + 8 * g;
        phf[u] = fa_b8(L.ph + o);
        plf[u] = fa_b8(L.pl + o);
        shf[u] = fa_b8(L.sh + o);
        slf[u] = fa_b8(L.sl + o);
      }
#pragma unroll
      for (int cc = 0; cc < NH; cc++) {
        const int o = (16 * (NH * wh + cc) + li) * LDT + 8 * g;
        const bf8 doh = fa_b8(L.dth + o), dol = fa_b8(L.dtl + o);
        const bf8 qh2 = fa_b8(L.qth + o), ql2 = fa_b8(L.qtl + o);
#pragma unroll
        for (int u = 0; u < 2; u++) {
          dv[u][cc] = mfma_bf16(phf[u], doh, dv[u][cc]);
          dv[u][cc] = mfma_bf16(plf[u], doh, dv[u][cc]);
          dv[u][cc] = mfma_bf16(phf[u], dol, dv[u][cc]);
          dk[u][cc] = mfma_bf16(shf[u], qh2, dk[u][cc]);
          dk[u][cc] = mfma_bf16(slf[u], qh2, dk[u][cc]);
          dk[u][cc] = mfma_bf16(shf[u], ql2, dk[u][cc]);
        }
      }
    }
    __syncthreads();
    st = st2;
  }
  if (it.slot < 0) {
#pragma unroll
    for (int u = 0; u < 2; u++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int key = c0 + 16 * u + 4 * g + i;
        if (key >= a.t) continue;
        float* kr = a.dk + (int64_t)key * a.ldk + (int64_t)kvh * HD + 16 * NH * wh + li;
        float* vr = a.dv + (int64_t)key * a.ld_dv + (int64_t)kvh * HD + 16 * NH * wh + li;
#pragma unroll
        for (int c = 0; c < NH; c++) {
          kr[16 * c] = dk[u][c][i];
          vr[16 * c] = dv[u][c][i];
        }
      }
  } else {  // 16-key sub-block 2 wk + u of the item -> its slot (dk rows, then dv rows); this wave's column half
#pragma unroll
    for (int u = 0; u < 2; u++) {
      float* pp = a.part + (int64_t)(it.slot + (2 * wk + u) * it.pad0) * (32 * HD) + 16 * NH * wh + li;
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int c = 0; c < NH; c++) {
          pp[(4 * g + i) * HD + 16 * c] = dk[u][c][i];
          pp[16 * HD + (4 * g + i) * HD + 16 * c] = dv[u][c][i];
        }
    }
  }
}

// ------------------------------------------------------------------ entry points: one workgroup per item
#define RTQ_FA_KERNEL(NAME, FN, LDS, HD)                                      \
  extern "C" __global__ __launch_bounds__(256) void NAME(MAttnArgs a) {       \
    __shared__ __attribute__((aligned(16))) LDS<HD> L;                        \
    if ((int)blockIdx.x >= a.n_items) return; /* whole workgroup */           \
    FN<HD>(a, a.items[blockIdx.x], L);                                        \
  }
RTQ_FA_KERNEL(rtq_m_fa_fwd64, fa_fwd, FaFwdLds, 64)
RTQ_FA_KERNEL(rtq_m_fa_fwd128, fa_fwd, FaFwdLds, 128)
#undef RTQ_FA_KERNEL

// the backward: the dk / dv items (the longer ones) then the dq items in one launch, each kind with
// its own partial slots; LDS sized for the larger of the two layouts
template <int HD>
union FaBwdLds {
  FaDqLds<HD> dq;
  FaKvLds<HD> kv;
};
#define RTQ_FA_BWD_KERNEL(NAME, HD)                                            \
  extern "C" __global__ __launch_bounds__(256) void NAME(MAttnArgs a) {       \
    __shared__ __attribute__((aligned(16))) FaBwdLds<HD> L;                   \
    const int b = (int)blockIdx.x;                                            \
    if (b < a.n_items2) {                                                     \
      MAttnArgs k = a;                                                        \
      k.part = a.part2;                                                       \
      fa_dkv<HD>(k, a.items2[b], L.kv);                                       \
    } else if (b < a.n_items2 + a.n_items) {                                  \
      fa_dq<HD>(a, a.items[b - a.n_items2], L.dq);                            \
    }                                                                         \
  }
RTQ_FA_BWD_KERNEL(rtq_m_fa_bwd64, 64)
RTQ_FA_BWD_KERNEL(rtq_m_fa_bwd128, 128)
#undef RTQ_FA_BWD_KERNEL
