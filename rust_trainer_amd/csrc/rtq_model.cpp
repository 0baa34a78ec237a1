// rtq_model.cpp — the device-resident training step over the frozen linears (rtq_model_* in
// include/rtq.h): a GGUF Qwen / Llama decoder loaded into HBM, LoRA adapters on its projections,
// and Model::forward_backward (src/model.rs:615-687) with every activation kept on the device.
//
// Reference structure restated (files under the reference repository):
//   load_gguf_from        src/rie.rs:164-260 (tensor names, tied head, kv_f16, QK-norm detection)
//   Model::attach_lora    src/model.rs:406-419, Lora::new src/linear.rs:21-25 (A ~ U(+-1/sqrt(in)), B = 0)
//   forward_backward      src/model.rs:644-687 (embed, blocks, head, blocks in reverse)
//   Block / Attention / Mlp src/model.rs:165-197, src/attention.rs:162-367, src/model.rs:113-134
// The reference recomputes each block's forward in the backward (checkpointing, src/model.rs:
// 663-665, 678-680) to save memory; the recomputation reproduces the same values.  Here the step
// keeps every block's activations when they fit (config-3 shapes: 60 MB per layer) and recomputes
// otherwise, or as rtq_model_set_checkpointing forces.
//
// Packed batches (Model::forward_backward_packed, src/model.rs:634-642): RoPE tables at the given
// token positions and the segment may-attend rule (Rope::allowed, src/ops.rs:160-167), applied as a
// 64 x 64 block liveness map (the attention products skip dead tiles and k slabs) plus the
// element rule in the softmax kernels.
//
// Linears that read the same input and share a ggml type run as one frozen weight: q | k | v
// (rows concatenated) and gate | up.  Their adapters become one LoRA of rank (members x r) whose B
// is block-diagonal (zeros elsewhere) and whose alpha is scaled alike, so alpha / rank and every
// output are unchanged; the gradients of the structurally zero B entries are cleared after each
// backward.  Each member adapter stays addressable (rtq_model_lora_*), its B as a strided block.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "rtq_internal.h"
#include "rtq_kargs.h"

namespace {

enum { LQ, LK, LV, LO, LGATE, LUP, LDOWN, NLIN };
const char* const kLinName[NLIN] = {"attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"};

#define M_TRY(expr)              \
  do {                           \
    rtq_status s_ = (expr);      \
    if (s_ != RTQ_OK) return s_; \
  } while (0)
#define M_HIP(expr)                                                                                     \
  do {                                                                                                  \
    hipError_t e_ = (expr);                                                                             \
    if (e_ != hipSuccess) return rtq_fail(RTQ_ERR_HIP, "%s: %s", #expr, hipGetErrorString(e_));         \
  } while (0)

// one member linear of a group: its rows of the fused weight and its adapter block
struct Member {
  int lin = 0;
  int64_t row0 = 0, rows = 0;
  int64_t col0 = 0, r = 0;  // adapter block: A rows / B columns [col0, col0 + r); r = 0: not adapted
};

// one frozen weight run by one linear call: a single linear, or q | k | v / gate | up fused
struct Group {
  rtq_weight* w = nullptr;
  const float* bias = nullptr;  // device [rows], or null
  int64_t rows = 0, in = 0;
  int nm = 0;
  Member mem[3];
  int64_t rank = 0;  // fused adapter rank (sum of the members' r); 0: no adapter
  float alpha = 0.0f;
  float *A = nullptr, *B = nullptr, *ga = nullptr, *gb = nullptr;  // [rank x in], [rows x rank]
  float* hpk = nullptr;  // the forward's LoRA-down partials of this step, reused by the backward (or null)
};

struct Layer {
  const float *attn_norm = nullptr, *ffn_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
  std::vector<Group> groups;
  int gi[NLIN], mi[NLIN];  // group and member of each linear
  bool qkv_fused = false, gu_fused = false;
};

// activations of one block, kept for its backward.  qkv holds q | k | v per token when fused (row
// stride qd + 2 kd), else q [t x qd], then k, then v; gu likewise gate | up.
struct Cache {
  float *n1, *inv1, *qkv, *q, *k, *v, *q_inv, *k_inv, *P, *o, *h, *n2, *inv2, *gu, *hm;
  float* lse;  // fused attention: log-sum-exp per (head, query) [nh x t] (P is then not kept)
  // with the step's dA / dB deferred to its end (defer_lg): the block's gradients that those read -
  // of gate | up, q | k | v, the attention output's residual branch and the block input - kept
  // per layer (null otherwise: the step-wide buffers are reused block after block)
  float *dgu = nullptr, *dqkv = nullptr, *dh = nullptr, *gx = nullptr;
};

// SplitMix64 + uniform of the reference Rng (src/tensor.rs:155-180)
struct Rng {
  uint64_t s;
  explicit Rng(uint64_t seed) : s(seed ^ 0x9E3779B97F4A7C15ULL) {}
  uint64_t next() {
    s += 0x9E3779B97F4A7C15ULL;
    uint64_t z = s;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
  }
  float uniform() { return (float)(next() >> 40) / (float)(1u << 24); }
  float uniform_sym(float bound) { return (uniform() * 2.0f - 1.0f) * bound; }
};

}  // namespace

struct rtq_model {
  rtq_ctx* ctx = nullptr;
  rtq_model_config cfg{};
  rtq_weight* embed = nullptr;
  rtq_weight* head = nullptr;  // == embed when tied
  const float* out_norm = nullptr;
  std::vector<Layer> layers;
  std::vector<void*> owned;  // device allocations of weights, norms, biases and adapters
  std::vector<rtq_weight*> weights;
  // step buffers, sized for t_cap tokens and n_cap targets
  int64_t t_cap = 0, n_cap = 0;
  void* step_mem = nullptr;
  void* grads = nullptr;  // every adapter's dA and dB (attach_lora), grad_bytes long
  size_t grad_bytes = 0;
  void* hpk_mem = nullptr;  // every group's kept LoRA-down partials
  size_t hpk_cap = 0;
  // each adapted group's h and g [t x rank] of one block's backward, kept from its dx kernel to
  // the block's one dA / dB launch (slot = group index within a layer, shared by the layers);
  // lora_batch false (RTQ_LORA_BATCH=0 at load time): dA / dB launched per linear, for comparison
  void* lg_mem = nullptr;
  size_t lg_cap = 0;
  std::vector<float*> lg_h, lg_g;  // slot (layer if deferring, else 0) * lg_groups + group
  int64_t lg_groups = 0;
  bool lora_batch = true;
  // norm_fuse: a block's two RMSNorms formed by the next linear's activation kernel where the shape
  // allows (RTQ_NORM_FUSE=0 at load time: the norm kernel, then the linear)
  bool norm_fuse = true;
  // defer_lg: every block's dA / dB left to one launch after the backward (their inputs kept per
  // layer: h / g slots per (layer, group), Cache gradient buffers), where the activations are kept
  // and the per-layer gradients fit a budget; RTQ_LORA_DEFER=0 at load time keeps per-block launches.
  // The job table and its workgroup map live in device memory, uploaded when they change.
  bool lora_defer = true, defer_lg = false;
  int64_t layout_defer = -1;  // defer_lg the step buffers were laid out for
  std::vector<LoraGradArgs> lg_all;
  void *lgt_mem = nullptr, *lgt_host = nullptr;
  size_t lgt_cap = 0, lgt_bytes = 0;
  std::vector<uintptr_t> lgt_key;  // the jobs' pointers and sizes when the table was last uploaded
  float *X = nullptr, *cos_ = nullptr, *sin_ = nullptr;
  std::vector<Cache> cache;
  int64_t cache_cap = 0;      // Cache sets allocated (n_layer when keeping, 1 when recomputing)
  int ckpt_mode = -1;         // -1 automatic, 0 keep activations, 1 recompute (rtq_model_set_checkpointing)
  bool ckpt = false;          // this step recomputes each block's forward in the backward
  std::vector<float> rope_factors;  // rope_freqs.weight (per-frequency divisors), or empty
  // packed layout of the current step (null / 0: a plain causal sequence)
  int32_t* seg_d = nullptr;
  uint8_t* live_d = nullptr;
  int64_t nlb = 0;
  bool packed = false;
  bool rope_plain = false;  // the uploaded RoPE tables are for positions 0..rope_t-1
  // fused attention (head_dim 64 or 128): work tables of the current layout, partial slots.
  // attn_mode -1 (default) and 1: fused whenever the head size allows (measured on the
  // Qwen3-0.6B-shaped step from 128 to 2048 tokens it ties or beats the probability-matrix path,
  // which 0 forces; rtq_model_set_attention).  attn_fused: this step's choice.
  bool attn_hd_ok = false;
  int attn_mode = -1;
  bool attn_fused = false;
  // the probability-matrix path's products on split 16-bit MFMA (rtq_m_gemm*_hf forward, *_bf
  // backward); RTQ_ATTN_F32=1 at load time keeps them on f32 MFMA (rtq_m_gemm*), for comparison
  bool attn_f32 = false;
  // fused attention: long query rows cut into pieces (attn_piece) and dk / dv ranges into pieces
  // aiming at attn_items work items per CU (RTQ_ATTN_ITEMS; 0: nothing is cut)
  int attn_items = 2;
  int64_t layout_fused = -1;  // attn_fused the step buffers were laid out for
  float* attn_D = nullptr;  // [nh x t] dO . o per query row
  uint16_t* attn_planes = nullptr;  // the fused backward's 16-bit operand planes (MAttnArgs::p*)
  void* attn_mem = nullptr;
  size_t attn_cap = 0;
  MAttnItem *it_fwd = nullptr, *it_kv = nullptr;
  MAttnMerge *mg_fwd = nullptr, *mg_kv = nullptr;
  int32_t *qmi = nullptr, *kmi = nullptr;  // (head, 16-row block) -> index into mg_fwd / mg_kv, or -1
  int n_fwd = 0, n_kv = 0, n_mfwd = 0, n_mkv = 0;
  float* attn_part = nullptr;     // forward and dq partial slots
  float* attn_part_kv = nullptr;  // dk / dv partial slots
  int64_t attn_t = -1;
  bool attn_packed = false;
  std::vector<int32_t> attn_seg;  // the segments the tables were built for
  // packed layouts: the forward attention over each segment's logical sequence (MSeqArgs): the
  // sequences' rows gathered back to back (gmap: packed row of each gathered row; sidx: each
  // packed row's own copy), the gathered q, k, v, o (and lse), and for the fused kernels the
  // sequences' items, merges and partial slots.  seq_on: this layout's forward runs that way
  // (off when the gathered rows would exceed 4 t + 64 per sequence: the packed rows' own tiles)
  struct SeqRun {
    int64_t base, len;
  };
  std::vector<SeqRun> seqs;
  std::vector<int32_t> seq_seg;  // the segments the sequences were built for
  bool seq_on = false, seq_fused = false;
  int64_t tv = 0;
  void* seq_mem = nullptr;
  size_t seq_cap = 0;
  int32_t *gmap_d = nullptr, *sidx_d = nullptr;
  float *gq = nullptr, *gk = nullptr, *gv = nullptr, *go = nullptr, *glse = nullptr, *seq_part = nullptr;
  MAttnItem* it_seq = nullptr;
  MAttnMerge* mg_seq = nullptr;
  int n_sit = 0, n_smg = 0;
  bool seq_pass = false;  // a sequence's unfused forward is running: its products take no liveness map
  // rtq_model_debug_capture: one layer's tensors copied during the step
  int64_t dbg_layer = -1;
  std::vector<std::pair<std::string, std::pair<float*, int64_t>>> dbg;
  float *dY, *dX, *mo, *f, *dhm, *dgu, *dn2, *dxu, *dh, *d_o, *dP, *dq, *dkh, *dvh, *dk, *dqkv, *dn1, *dxk, *dxv;
  int32_t *tok_d = nullptr, *pos_d = nullptr, *tgt_d = nullptr, *hit_d = nullptr;
  float *wts_d = nullptr, *logp_d = nullptr;
  int64_t rope_t = -1;  // t of the uploaded RoPE tables
  // the step's kernels as one HIP graph (RTQ_STEP_GRAPH=0 at load: every step eager).  A step
  // whose launch key (sizes, choices, plan counts, gen and the context's workspace generation)
  // equals the previous step's is captured; later steps with that key replay it.  gen is bumped
  // by everything else a launch's arguments depend on: a (re)allocation, a rebuilt attention plan,
  // new adapters, a setter.
  bool graph_on = true;
  hipGraphExec_t gexec = nullptr;
  std::vector<uint64_t> gkey, prev_key;
  uint64_t gen = 0;
  int64_t graph_replays = 0;
  // pinned staging of the step's host inputs (tokens, target positions and tokens, weights) and
  // outputs (log-probs, hits)
  void* io_host = nullptr;
  size_t io_cap = 0;
};

namespace {

rtq_status dev_alloc(rtq_model* m, size_t bytes, void** out) {
  M_HIP(hipMalloc(out, bytes ? bytes : 4));
  m->owned.push_back(*out);
  m->gen++;
  return RTQ_OK;
}

void dev_free(rtq_model* m, void* p) {
  if (!p) return;
  for (size_t i = 0; i < m->owned.size(); i++)
    if (m->owned[i] == p) {
      m->owned.erase(m->owned.begin() + (ptrdiff_t)i);
      (void)hipFree(p);
      m->gen++;
      return;
    }
}

rtq_status upload_vec(rtq_model* m, const rtq_gguf* g, const std::string& name, int64_t n, const float** out,
                      bool required) {
  *out = nullptr;
  const int64_t i = rtq_gguf_find_tensor(g, name.c_str());
  if (i < 0) return required ? rtq_fail(RTQ_ERR_INVALID, "GGUF: missing tensor %s", name.c_str()) : RTQ_OK;
  int type = 0, nd = 0;
  int64_t ne[4];
  const void* data = nullptr;
  size_t nbytes = 0;
  M_TRY(rtq_gguf_tensor(g, i, nullptr, &type, &nd, ne, &data, &nbytes));
  if (type != RTQ_TYPE_F32 || nbytes != (size_t)n * 4)
    return rtq_fail(RTQ_ERR_UNSUPPORTED, "GGUF: %s must be F32 with %lld elements", name.c_str(), (long long)n);
  void* d;
  M_TRY(dev_alloc(m, nbytes, &d));
  M_HIP(hipMemcpy(d, data, nbytes, hipMemcpyHostToDevice));
  *out = (const float*)d;
  return RTQ_OK;
}

double kv_num(const rtq_gguf* g, const std::string& key, double dflt) {
  double v = 0.0;
  return rtq_gguf_get_f64(g, key.c_str(), &v) == RTQ_OK ? v : dflt;
}

rtq_status load_weight(rtq_model* m, const rtq_gguf* g, const std::string& name, int64_t out, int64_t in,
                       rtq_weight** w) {
  M_TRY(rtq_weight_from_gguf(m->ctx, g, name.c_str(), w));
  m->weights.push_back(*w);
  if (rtq_weight_out_dim(*w) != out || rtq_weight_in_dim(*w) != in)
    return rtq_fail(RTQ_ERR_INVALID, "GGUF: %s is %lldx%lld, expected %lldx%lld", name.c_str(),
                    (long long)rtq_weight_out_dim(*w), (long long)rtq_weight_in_dim(*w), (long long)out, (long long)in);
  return RTQ_OK;
}

hipStream_t stream_of(rtq_model* m) { return (hipStream_t)rtq_ctx_stream(m->ctx); }

// ---------------------------------------------------------------- launches
rtq_status k_norm(rtq_model* m, const float* a, const float* b, float* h, const float* w, float* y, float* inv,
                  int64_t rows, int64_t d, int fused) {
  // a wave per row where the row fits the wave layout (one-wave workgroups, no barrier)
  const bool wave = d % 256 == 0 && d <= 2048 && ((uintptr_t)a | (uintptr_t)b | (uintptr_t)h | (uintptr_t)w |
                                                   (uintptr_t)y) % 16 == 0;
  MNormArgs na{a, b, h, w, y, inv, (int)rows, (int)d, m->cfg.rms_eps, m->cfg.norm_offset, fused, wave ? 1 : 0};
  return rtq_model_launch(m->ctx, KM_RMSNORM, dim3((unsigned)rows), dim3(wave ? 64 : 256), stream_of(m), &na);
}

rtq_status k_norm_bwd(rtq_model* m, const float* x, const float* w, const float* inv, const float* dy, const float* res,
                      float* out, int64_t rows, int64_t d) {
  const bool wave = d % 256 == 0 && d <= 2048 && ((uintptr_t)x | (uintptr_t)w | (uintptr_t)dy | (uintptr_t)res |
                                                   (uintptr_t)out) % 16 == 0;
  MNormBwdArgs na{x, w, inv, dy, res, out, (int)rows, (int)d, m->cfg.norm_offset, wave ? 1 : 0};
  return rtq_model_launch(m->ctx, KM_RMSNORM_BWD, dim3((unsigned)rows), dim3(wave ? 64 : 256), stream_of(m), &na);
}

// elementwise over rows x cols (a, b at row stride lda, c at ldc, y, z at ldy)
rtq_status k_elt2(rtq_model* m, int km, const float* a, const float* b, const float* c, float* y, float* z,
                  int64_t rows, int64_t cols, int64_t lda, int64_t ldc, int64_t ldy) {
  MEltArgs ea{a, b, c, y, z, rows * cols, cols, lda, ldc, ldy};
  const unsigned grid = (unsigned)std::min<int64_t>((rows * cols + 255) / 256, 4096);
  return rtq_model_launch(m->ctx, km, dim3(grid), dim3(256), stream_of(m), &ea);
}

rtq_status k_elt(rtq_model* m, int km, const float* a, const float* b, const float* c, float* y, float* z, int64_t n) {
  return k_elt2(m, km, a, b, c, y, z, 1, n, n, n, n);
}

struct Op {  // one GEMM operand: base, batch stride and divisor, row / column strides
  const float* p;
  int64_t sb, s0, s1;
  int div;
};

// C(b, m, n) (+)= sum_k A(b, m, k) B(b, k, n) for b < batch
// attention products of the step take the packed layout's liveness map (null for a plain sequence)
// split: the 16-bit MFMA form of the product (rtq_m_gemm*_hf for the forward's, rtq_m_gemm*_bf for
// the backward's), unless attn_f32 keeps every product on f32 MFMA
enum GemmSplit { SPLIT_HF, SPLIT_BF };
rtq_status k_gemm(rtq_model* m, int64_t M, int64_t N, int64_t K, int64_t batch, Op A, Op B, float* C, int64_t sCb,
                  int64_t sCm, int64_t sCn, float a_scale, int causal, int acc, GemmSplit split) {
  MGemmArgs ga{A.p, B.p, C, (int)M, (int)N, (int)K, A.sb, A.s0, A.s1, B.sb, B.s0, B.s1, sCb, sCm, sCn, A.div, B.div,
               a_scale, causal, acc, (int)batch, causal && m->packed && !m->seq_pass ? m->live_d : nullptr,
               (int)m->nlb, nullptr};
  // 64-row tiles when the grid fills the chip twice over, else 32-row tiles (twice the workgroups)
  const int64_t tiles64 = (N + 63) / 64 * ((M + 63) / 64) * batch / (causal == 1 ? 2 : 1);
  const int bm = tiles64 >= 2 * 256 ? 64 : 32;
  const int64_t tiles = (N + 63) / 64 * ((M + bm - 1) / bm) * batch;  // flat, XCD-aware (8 x ceil(tiles / 8))
  const int kid = m->attn_f32          ? (bm == 64 ? KM_GEMM : KM_GEMM32)
                  : split == SPLIT_HF ? (bm == 64 ? KM_GEMM_HF : KM_GEMM32_HF)
                                      : (bm == 64 ? KM_GEMM_BF : KM_GEMM32_BF);
  return rtq_model_launch(m->ctx, kid, dim3((unsigned)((tiles + 7) / 8 * 8)), dim3(256), stream_of(m), &ga);
}

// independent products C_i (+)= A_i B_i (M_i x N_i x K_i, batch_i) in one launch of 32-row tiles
struct GemmJob {
  int64_t M, N, K, batch;
  Op A, B;
  float* C;
  int64_t sCb, sCm, sCn;
  float a_scale;
  int causal, acc;
};
rtq_status k_gemm_group(rtq_model* m, const GemmJob* jobs, int n) {
  if (n < 1 || n > 3) return rtq_fail(RTQ_ERR_INVALID, "internal: %d grouped products", n);
  MGemmGroupArgs g{};
  g.np = n;
  int64_t total = 0;
  for (int i = 0; i < n; i++) {
    const GemmJob& j = jobs[i];
    g.p[i] = MGemmArgs{j.A.p, j.B.p, j.C, (int)j.M, (int)j.N, (int)j.K, j.A.sb, j.A.s0, j.A.s1, j.B.sb, j.B.s0,
                       j.B.s1, j.sCb, j.sCm, j.sCn, j.A.div, j.B.div, j.a_scale, j.causal, j.acc, (int)j.batch,
                       j.causal && m->packed ? m->live_d : nullptr, (int)m->nlb, nullptr};
    g.start[i] = (int)total;
    total += (j.N + 63) / 64 * ((j.M + 31) / 32) * j.batch;
  }
  for (int i = n; i < 4; i++) g.start[i] = (int)total;
  return rtq_model_launch(m->ctx, m->attn_f32 ? KM_GEMM32G : KM_GEMM32G_BF, dim3((unsigned)((total + 7) / 8 * 8)),
                          dim3(256), stream_of(m), &g);
}

rtq_lora lora_view(const Group& l) { return rtq_lora{l.rank, l.alpha, l.A, l.B, l.rank > 0 ? 1 : 0}; }

// a fused group's members as rank blocks (nm 0: one plain adapter)
RankBlocks rank_blocks(const Group& l) {
  RankBlocks rb{};
  if (l.nm < 2) return rb;
  rb.nm = l.nm;
  for (int i = 0; i < l.nm; i++) {
    rb.row0[i] = (int)l.mem[i].row0;
    rb.nrow[i] = (int)l.mem[i].rows;
    rb.col0[i] = (int)l.mem[i].col0;
    rb.r[i] = (int)l.mem[i].r;
  }
  return rb;
}

rtq_status lin_fwd(rtq_model* m, const Group& l, const float* x, int64_t t, float* y) {
  const rtq_lora lv = lora_view(l);
  const RankBlocks rb = rank_blocks(l);
  return rtq_linear_forward_keep_d(m->ctx, l.w, l.bias, l.rank > 0 ? &lv : nullptr, &rb, x, t, y, l.hpk,
                                   stream_of(m));
}

// n = rmsnorm(a (+ b)) (h = a + b, inv = 1 / rms), then y = the linear of n: the linear's activation
// kernel forms n where the shape allows (the same bits as the norm kernel's one-wave rows), else
// the norm kernel runs first.  n, h and inv are written either way.
rtq_status lin_fwd_norm(rtq_model* m, const Group& l, const float* a, const float* b, float* h, const float* nw,
                        float* n, float* inv, int64_t t, float* y) {
  const NormIn ni{a, b, h, nw, inv, m->cfg.rms_eps, m->cfg.norm_offset};
  if (m->norm_fuse && rtq_norm_fusable(l.w, ni, n)) {
    const rtq_lora lv = lora_view(l);
    const RankBlocks rb = rank_blocks(l);
    return rtq_linear_forward_norm_d(m->ctx, l.w, l.bias, l.rank > 0 ? &lv : nullptr, &rb, &ni, n, t, y, l.hpk,
                                     stream_of(m));
  }
  M_TRY(k_norm(m, a, b, h, nw, n, inv, t, m->cfg.n_embd, 0));
  return lin_fwd(m, l, n, t, y);
}

// the down projection of SwiGLU's hm = silu(g) * u (src/model.rs:124-125): quantised weights form hm
// in their activation kernel (one launch less); dense ones, or operands off 16-byte alignment, run
// the elementwise kernel first.  hm is written either way (the backward reads it).
rtq_status lin_fwd_swiglu(rtq_model* m, const Group& l, const float* g, const float* u, int64_t ldg, float* hm,
                          int64_t t, float* y) {
  const int64_t ff = m->cfg.n_ff;
  const int wt = rtq_weight_type(l.w);
  const bool aligned = ldg % 4 == 0 && ((uintptr_t)g | (uintptr_t)u | (uintptr_t)hm) % 16 == 0;
  if (wt != RTQ_TYPE_F32 && wt != RTQ_TYPE_TQ8_0 && aligned) {
    const rtq_lora lv = lora_view(l);
    const RankBlocks rb = rank_blocks(l);
    return rtq_linear_forward_swiglu_d(m->ctx, l.w, l.bias, l.rank > 0 ? &lv : nullptr, &rb, g, u, ldg, hm, t, y,
                                       l.hpk, stream_of(m));
  }
  M_TRY(k_elt2(m, KM_SWIGLU, g, u, nullptr, hm, nullptr, t, ff, ldg, ff, ff));
  return lin_fwd(m, l, hm, t, y);
}

// a fused group's adapter is block-diagonal (each member's rows see only its own ranks): the
// quantised backward computes gb and g = s dy.B inside the blocks only; the dense (f32 GEMM) one
// computes every pair and the off-block gb entries are cleared after it.  jobs (or null): a
// quantised adapted group's dA / dB are appended there (h, g in the group's slot gi) for the
// block's batched launch instead of being launched here.
// sw (or null): dx is SwiGLU's dh; where the deferred path runs, its finish writes sw's dg / du
// instead of dx and *sw_done is set (else dx is written and the caller runs the SwiGLU backward)
rtq_status lin_bwd(rtq_model* m, const Layer& L, int gi, const float* x, const float* dy, int64_t t, float* dx,
                   std::vector<LoraGradArgs>* jobs = nullptr, const SwiGluBwd* sw = nullptr, bool* sw_done = nullptr) {
  const Group& l = L.groups[(size_t)gi];
  const rtq_lora lv = lora_view(l);
  const int wt = rtq_weight_type(l.w);
  const bool dense = wt == RTQ_TYPE_F32 || wt == RTQ_TYPE_TQ8_0;
  if (sw_done) *sw_done = false;
  if (jobs && m->lora_batch && !dense && l.rank > 0 && jobs->size() < RTQ_LORA_JOBS) {
    const RankBlocks rb = rank_blocks(l);
    LoraGradArgs job{};
    const size_t slot = (size_t)(m->defer_lg ? &L - m->layers.data() : 0) * (size_t)m->lg_groups + (size_t)gi;
    M_TRY(rtq_linear_backward_defer_d(m->ctx, l.w, &lv, l.nm < 2 ? nullptr : &rb, x, dy, t, dx, l.ga, l.gb, l.hpk,
                                      m->lg_h[slot], m->lg_g[slot], &job, stream_of(m), sw));
    jobs->push_back(job);
    if (sw_done) *sw_done = sw != nullptr;
    return RTQ_OK;
  }
  if (l.rank == 0 || dense)
    M_TRY(rtq_linear_backward_d(m->ctx, l.w, l.rank > 0 ? &lv : nullptr, x, dy, t, dx, l.ga, l.gb, stream_of(m)));
  if (l.rank == 0 || (dense && l.nm < 2)) return RTQ_OK;
  if (!dense && l.nm < 2)
    return rtq_linear_backward_blocks_d(m->ctx, l.w, &lv, nullptr, x, dy, t, dx, l.ga, l.gb, l.hpk, stream_of(m));
  if (!dense) {
    const RankBlocks rb = rank_blocks(l);
    return rtq_linear_backward_blocks_d(m->ctx, l.w, &lv, &rb, x, dy, t, dx, l.ga, l.gb, l.hpk, stream_of(m));
  }
  MMaskArgs ma{l.gb, l.rows, l.rank, l.nm, {}, {}, {}, {}};
  for (int i = 0; i < l.nm; i++) {
    ma.row0[i] = l.mem[i].row0;
    ma.nrow[i] = l.mem[i].rows;
    ma.col0[i] = l.mem[i].col0;
    ma.r[i] = l.mem[i].r;
  }
  return rtq_model_launch(m->ctx, KM_LORA_MASK, dim3((unsigned)std::min<int64_t>((l.rows * l.rank + 255) / 256, 4096)),
                          dim3(256), stream_of(m), &ma);
}

// ---------------------------------------------------------------- step buffers
// one buffer for every adapted group's kept LoRA-down partials at t tokens (rank and t may change
// between steps: sized and assigned per step)
rtq_status ensure_hpk(rtq_model* m, int64_t t) {
  size_t need = 0;
  for (auto& L : m->layers)
    for (auto& G : L.groups) need += ((size_t)rtq_lora_partial_floats(G.w, t, G.rank) * 4 + 255) / 256 * 256;
  if (need > m->hpk_cap) {
    if (m->hpk_mem) {
      M_HIP(hipStreamSynchronize(stream_of(m)));
      M_HIP(hipFree(m->hpk_mem));
      m->hpk_mem = nullptr;
      m->hpk_cap = 0;
    }
    M_HIP(hipMalloc(&m->hpk_mem, need));
    m->hpk_cap = need;
    m->gen++;
  }
  char* p = (char*)m->hpk_mem;
  for (auto& L : m->layers)
    for (auto& G : L.groups) {
      const size_t f = (size_t)rtq_lora_partial_floats(G.w, t, G.rank);
      G.hpk = f ? (float*)p : nullptr;
      p += (f * 4 + 255) / 256 * 256;
    }
  return RTQ_OK;
}

// the h / g slots of the batched dA / dB launches (ensure_hpk's sizing rule: per step)
rtq_status ensure_lgrad(rtq_model* m, int64_t t) {
  std::vector<int64_t> rmax;
  for (auto& L : m->layers) {
    if (rmax.size() < L.groups.size()) rmax.resize(L.groups.size(), 0);
    for (size_t i = 0; i < L.groups.size(); i++) rmax[i] = std::max(rmax[i], L.groups[i].rank);
  }
  const int64_t nl = m->defer_lg ? m->cfg.n_layer : 1;  // slot sets: one per layer when deferring
  size_t per = 0;
  for (int64_t r : rmax) per += ((size_t)(2 * t * r) * 4 + 255) / 256 * 256;
  const size_t need = per * (size_t)nl;
  if (need > m->lg_cap) {
    if (m->lg_mem) {
      M_HIP(hipStreamSynchronize(stream_of(m)));
      M_HIP(hipFree(m->lg_mem));
      m->lg_mem = nullptr;
      m->lg_cap = 0;
    }
    M_HIP(hipMalloc(&m->lg_mem, need));
    m->lg_cap = need;
    m->gen++;
  }
  m->lg_groups = (int64_t)rmax.size();
  m->lg_h.assign((size_t)nl * rmax.size(), nullptr);
  m->lg_g.assign((size_t)nl * rmax.size(), nullptr);
  char* p = (char*)m->lg_mem;
  for (int64_t l = 0; l < nl; l++)
    for (size_t i = 0; i < rmax.size(); i++) {
      m->lg_h[(size_t)l * rmax.size() + i] = (float*)p;
      m->lg_g[(size_t)l * rmax.size() + i] = (float*)p + t * rmax[i];
      p += ((size_t)(2 * t * rmax[i]) * 4 + 255) / 256 * 256;
    }
  return RTQ_OK;
}

// halves of the fused backward's operand planes for T tokens: natural q scale (2), dO (2), k (1),
// v (2) planes of [T][heads][hd]; transposed q (2), dO (2), k (2) planes of [heads][hd][T rounded
// up to 64]
int64_t attn_plane_halves(const rtq_model_config& c, int64_t T) {
  const int64_t qd = c.n_head * c.head_dim, kd = c.n_head_kv * c.head_dim, tp = (T + 63) / 64 * 64;
  return T * (4 * qd + 3 * kd) + tp * (4 * qd + 2 * kd);
}

// Assigns every step buffer of `dst` for T tokens, N targets and `caches` sets of block activations
// (n_layer when keeping them, 1 when recomputing) from `base` (0: only counts) and returns the
// bytes.  Each buffer starts on a 256-byte boundary.
size_t step_layout(rtq_model* dst, int64_t T, int64_t N, int64_t caches, uintptr_t base) {
  const rtq_model_config& c = dst->cfg;
  const int64_t d = c.n_embd, qd = c.n_head * c.head_dim, kd = c.n_head_kv * c.head_dim, ff = c.n_ff;
  const int64_t half = c.rope_dim / 2, L = c.n_layer;
  // the unfused attention keeps P [nh x t x t] per layer and needs dP and per-head dk, dv; the
  // fused kernels keep only each row's log-sum-exp
  const bool fz = dst->attn_fused;
  const int64_t att = fz ? 1 : c.n_head * T * T, hdh = fz ? 1 : c.n_head * T * c.head_dim, nlb = (T + 63) / 64;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const uintptr_t p = base + off;
    off += (bytes + 255) / 256 * 256;
    return p;
  };
  auto fl = [&](float** p, int64_t floats) { *p = reinterpret_cast<float*>(take((size_t)floats * 4)); };
  fl(&dst->X, (L + 1) * T * d);
  fl(&dst->cos_, T * half + 1);
  fl(&dst->sin_, T * half + 1);
  dst->cache.assign((size_t)caches, Cache{});
  for (Cache& k : dst->cache) {
    fl(&k.n1, T * d), fl(&k.inv1, T), fl(&k.qkv, T * (qd + 2 * kd)), fl(&k.q, T * qd), fl(&k.k, T * kd);
    fl(&k.v, T * kd), fl(&k.q_inv, T * c.n_head), fl(&k.k_inv, T * c.n_head_kv), fl(&k.P, att), fl(&k.o, T * qd);
    fl(&k.h, T * d), fl(&k.n2, T * d), fl(&k.inv2, T), fl(&k.gu, T * 2 * ff), fl(&k.hm, T * ff);
    fl(&k.lse, fz ? c.n_head * T : 1);
    if (dst->defer_lg) fl(&k.dgu, T * 2 * ff), fl(&k.dqkv, T * (qd + 2 * kd)), fl(&k.dh, T * d), fl(&k.gx, T * d);
  }
  fl(&dst->attn_D, fz ? c.n_head * T : 1);
  dst->attn_planes = reinterpret_cast<uint16_t*>(take((size_t)(fz ? attn_plane_halves(c, T) : 1) * 2));
  fl(&dst->dY, T * d), fl(&dst->dX, T * d), fl(&dst->mo, T * d), fl(&dst->f, T * d), fl(&dst->dhm, T * ff);
  fl(&dst->dgu, T * 2 * ff), fl(&dst->dn2, T * d), fl(&dst->dxu, T * d), fl(&dst->dh, T * d), fl(&dst->d_o, T * qd);
  fl(&dst->dP, att), fl(&dst->dq, T * qd), fl(&dst->dkh, hdh), fl(&dst->dvh, hdh), fl(&dst->dk, T * kd);
  fl(&dst->dqkv, T * (qd + 2 * kd)), fl(&dst->dn1, T * d), fl(&dst->dxk, T * d), fl(&dst->dxv, T * d);
  fl(&dst->wts_d, N), fl(&dst->logp_d, N);
  dst->tok_d = reinterpret_cast<int32_t*>(take((size_t)T * 4));
  dst->seg_d = reinterpret_cast<int32_t*>(take((size_t)T * 4));
  dst->live_d = reinterpret_cast<uint8_t*>(take((size_t)(nlb * nlb)));
  for (int32_t** q : {&dst->pos_d, &dst->tgt_d, &dst->hit_d}) *q = reinterpret_cast<int32_t*>(take((size_t)N * 4));
  return off;
}

// whether a step of t tokens recomputes block activations: as forced, or (automatic) when keeping
// every layer's activations would take more than half of the device memory free now
rtq_status choose_ckpt(rtq_model* m, int64_t t, int64_t n) {
  if (m->ckpt_mode >= 0) {
    m->ckpt = m->ckpt_mode == 1;
    return RTQ_OK;
  }
  if (m->cfg.n_layer <= 1) {
    m->ckpt = false;
    return RTQ_OK;
  }
  const int64_t T = std::max(t, m->t_cap), N = std::max<int64_t>(std::max(n, m->n_cap), 1);
  rtq_model probe;
  probe.cfg = m->cfg;
  probe.attn_fused = m->attn_fused;
  const size_t keep = step_layout(&probe, T, N, m->cfg.n_layer, 0);
  size_t free_b = 0, total_b = 0;
  M_HIP(hipMemGetInfo(&free_b, &total_b));
  const size_t held = m->step_mem ? step_layout(&probe, m->t_cap, std::max<int64_t>(m->n_cap, 1), m->cache_cap, 0) : 0;
  m->ckpt = keep > (free_b + held) / 2;
  return RTQ_OK;
}

// whether this step defers every block's dA / dB to one launch after the backward: activations
// kept, some adapter attached, and the per-layer gradient buffers within min(4 GiB, free / 4)
rtq_status choose_defer(rtq_model* m, int64_t t) {
  const rtq_model_config& c = m->cfg;
  bool adapted = false;
  for (const Layer& L : m->layers)
    for (const Group& g : L.groups) adapted = adapted || g.rank > 0;
  m->defer_lg = false;
  if (m->ckpt || !m->lora_batch || !m->lora_defer || !adapted || c.n_layer < 2) return RTQ_OK;
  const int64_t T = std::max(t, m->t_cap), qd = c.n_head * c.head_dim, kd = c.n_head_kv * c.head_dim;
  const size_t extra = (size_t)c.n_layer * (size_t)T * (size_t)(2 * c.n_ff + qd + 2 * kd + 2 * c.n_embd) * 4;
  size_t free_b = 0, total_b = 0;
  M_HIP(hipMemGetInfo(&free_b, &total_b));
  const size_t held = m->layout_defer == 1 ? extra : 0;  // already allocated: counts as free
  m->defer_lg = extra <= std::min<size_t>((size_t)4 << 30, (free_b + held) / 4);
  return RTQ_OK;
}

rtq_status ensure_step(rtq_model* m, int64_t t, int64_t n) {
  const int64_t caches = m->ckpt ? 1 : m->cfg.n_layer;
  if (t <= m->t_cap && n <= m->n_cap && caches == m->cache_cap && m->layout_fused == (int64_t)m->attn_fused &&
      m->layout_defer == (int64_t)m->defer_lg)
    return RTQ_OK;
  const int64_t T = std::max(t, m->t_cap), N = std::max<int64_t>(std::max(n, m->n_cap), 1);
  if (m->step_mem) {
    M_HIP(hipStreamSynchronize(stream_of(m)));
    M_HIP(hipFree(m->step_mem));
    m->step_mem = nullptr;
  }
  m->t_cap = m->n_cap = m->cache_cap = 0;
  const size_t bytes = step_layout(m, T, N, caches, 0);
  M_HIP(hipMalloc(&m->step_mem, bytes));
  step_layout(m, T, N, caches, reinterpret_cast<uintptr_t>(m->step_mem));
  m->t_cap = T;
  m->n_cap = N;
  m->cache_cap = caches;
  m->layout_fused = m->attn_fused;
  m->layout_defer = m->defer_lg;
  m->rope_t = -1;
  m->gen++;
  return RTQ_OK;
}

// RoPE tables for the tokens' positions (Rope::at_positions, src/ops.rs:141-167; positions null:
// 0..t-1), computed in f32 on the host: inverse frequencies base^(-2i / rot) * freq_scale, divided
// by rope_freqs.weight's factor where that is non-zero
rtq_status ensure_rope(rtq_model* m, int64_t t, const int32_t* positions) {
  if (!positions && m->rope_plain && m->rope_t == t) return RTQ_OK;
  const rtq_model_config& c = m->cfg;
  const int64_t half = c.rope_dim / 2;
  std::vector<float> cs((size_t)(t * half)), sn((size_t)(t * half));
  for (int64_t i = 0; i < half; i++) {
    float fr = powf(c.rope_base, -2.0f * (float)i / (float)c.rope_dim) * c.rope_freq_scale;
    if (i < (int64_t)m->rope_factors.size() && m->rope_factors[(size_t)i] != 0.0f) fr /= m->rope_factors[(size_t)i];
    for (int64_t p = 0; p < t; p++) {
      const float a = (float)(positions ? positions[p] : p) * fr;
      cs[(size_t)(p * half + i)] = cosf(a);
      sn[(size_t)(p * half + i)] = sinf(a);
    }
  }
  M_HIP(hipMemcpyAsync(m->cos_, cs.data(), cs.size() * 4, hipMemcpyHostToDevice, stream_of(m)));
  M_HIP(hipMemcpyAsync(m->sin_, sn.data(), sn.size() * 4, hipMemcpyHostToDevice, stream_of(m)));
  M_HIP(hipStreamSynchronize(stream_of(m)));  // the host tables go out of scope
  m->rope_t = t;
  m->rope_plain = positions == nullptr;
  return RTQ_OK;
}

// the packed layout's segments and 64 x 64 block liveness map (a block of (query, key) pairs is
// live when some pair may attend: the diagonal blocks always, an earlier key block when it holds a
// shared-prompt token or a segment that the query block holds too)
rtq_status upload_layout(rtq_model* m, const int32_t* seg, int64_t t) {
  if (!seg) {
    m->packed = false;
    m->nlb = 0;
    return RTQ_OK;
  }
  const int64_t nlb = (t + 63) / 64;
  std::vector<std::vector<int32_t>> segs((size_t)nlb);
  std::vector<uint8_t> has0((size_t)nlb, 0), live((size_t)(nlb * nlb), 0);
  for (int64_t b = 0; b < nlb; b++) {
    std::vector<int32_t>& v = segs[(size_t)b];
    for (int64_t j = b * 64; j < std::min(t, b * 64 + 64); j++) {
      if (seg[j] == 0) has0[(size_t)b] = 1;
      else v.push_back(seg[j]);
    }
    std::sort(v.begin(), v.end());
    v.erase(std::unique(v.begin(), v.end()), v.end());
  }
  for (int64_t a = 0; a < nlb; a++)
    for (int64_t b = 0; b <= a; b++) {
      bool lv = a == b || has0[(size_t)b];
      if (!lv) {
        const auto &x = segs[(size_t)a], &y = segs[(size_t)b];
        size_t i = 0, j = 0;
        while (!lv && i < x.size() && j < y.size()) {
          if (x[i] == y[j]) lv = true;
          else if (x[i] < y[j]) i++;
          else j++;
        }
      }
      live[(size_t)(a * nlb + b)] = lv ? 1 : 0;
    }
  M_HIP(hipMemcpyAsync(m->seg_d, seg, (size_t)t * 4, hipMemcpyHostToDevice, stream_of(m)));
  M_HIP(hipMemcpyAsync(m->live_d, live.data(), live.size(), hipMemcpyHostToDevice, stream_of(m)));
  M_HIP(hipStreamSynchronize(stream_of(m)));
  m->packed = true;
  m->nlb = nlb;
  return RTQ_OK;
}

// tiles per piece of query block qb's key range (the forward and dq items): 3 for the first eight
// blocks, 6 after (never cut with attn_items 0).  A rule of the block index alone, so that a query
// row's pieces, and so its bits, are the same at every sequence length and in a packed layout's
// logical sequences.  Measured on the Qwen3-0.6B-shaped step: shorter pieces cost more in merges
// than they gain, longer ones leave the longest rows as the tail (2048 tokens: 48.2 ms at 6 tiles,
// 52.0 uncut; 512: 12.98 at 3, 13.44 at 2).
int64_t attn_piece(const rtq_model* m, int64_t qb) {
  return m->attn_items > 0 ? (qb < 8 ? 3 : 6) : INT32_MAX;
}

// appends the items of one block (live tiles L, cut into pieces of `chunk`) of the sequence at
// rows [rbase, rbase + rlen): a block cut into n > 1 pieces takes 4 n slots, 16-row sub-block w of
// piece i writing slot s0 + i + w n, so each sub-block's n partials are contiguous (one merge each)
void attn_cut(const std::vector<int>& L, int64_t chunk, int head, int blk, int rbase, int rlen, int& slots,
              std::vector<MAttnItem>& items, std::vector<MAttnMerge>& merges) {
  const int n = (int)((L.size() + chunk - 1) / chunk);
  if (n == 0) return;
  const int s0 = n > 1 ? slots : -1;
  for (int i = 0; i < n; i++) {
    const int a0 = L[(size_t)(i * chunk)], a1 = L[std::min(L.size(), (size_t)((i + 1) * chunk)) - 1] + 1;
    items.push_back(MAttnItem{head, blk, a0, a1, n > 1 ? s0 + i : -1, n, rbase, rlen});
  }
  if (n > 1) {
    for (int w = 0; w < 4; w++)
      if ((4 * blk + w) * 16 < rlen) merges.push_back(MAttnMerge{head, 4 * blk + w, s0 + w * n, n, rbase, rlen});
    slots += 4 * n;
  }
}

// work tables of the fused attention for t tokens and the current layout (segments or null):
// forward / dq items (head, 16-row query block, range of its live 64-key tiles) and dk / dv items
// (KV head, 16-key block, range of its live (group head, 64-query tile) pairs), each block's list
// cut into chunks of at most `chunk` live tiles so that there are about three items per SIMD; blocks
// cut into several items get partial slots and a merge entry.  Rebuilt when t or the layout changes.
rtq_status ensure_attn_plan(rtq_model* m, int64_t t, const int32_t* seg) {
  const bool packed = seg != nullptr;
  if (m->attn_t == t && m->attn_packed == packed &&
      (!packed || std::equal(m->attn_seg.begin(), m->attn_seg.end(), seg)))
    return RTQ_OK;
  const rtq_model_config& c = m->cfg;
  const int nh = (int)c.n_head, nkv = (int)c.n_head_kv, grp = nh / nkv;
  const int64_t nkt = (t + 63) / 64, nlb = (t + 63) / 64;
  // the block liveness of the layout (as upload_layout derives it)
  std::vector<uint8_t> live;
  if (packed) {
    live.assign((size_t)(nlb * nlb), 0);
    M_HIP(hipMemcpy(live.data(), m->live_d, live.size(), hipMemcpyDeviceToHost));
  }
  auto lv = [&](int64_t qb64, int64_t kb64) { return kb64 <= qb64 && (!packed || live[(size_t)(qb64 * nlb + kb64)]); };
  // items of 64 rows (one workgroup of four waves each): a query block's live key tiles (forward,
  // dq), a key block's live (group head, query tile) pairs (dk, dv)
  std::vector<std::vector<int>> fl((size_t)nlb), kl((size_t)nlb);
  int64_t ku = 0;
  for (int64_t qb = 0; qb < nlb; qb++)
    for (int64_t kt = 0; kt <= qb; kt++)
      if (lv(qb, kt)) fl[(size_t)qb].push_back((int)kt);
  for (int64_t kb = 0; kb < nlb; kb++) {
    for (int hr = 0; hr < grp; hr++)
      for (int64_t qt = kb; qt < nkt; qt++)
        if (lv(qt, kb)) kl[(size_t)kb].push_back((int)(hr * nkt + qt));
    ku += (int64_t)kl[(size_t)kb].size() * nkv;
  }
  // dk / dv ranges are cut into pieces (partials merged after) of about the length that gives
  // attn_items workgroups per CU, kept within 3 .. 6 tiles; query blocks by attn_piece (a rule of
  // the block index alone).  attn_items 0: no cuts, no merges.
  const int64_t target = (int64_t)m->attn_items * rtq_ctx_cu_count(m->ctx);
  const int64_t ck = target > 0 ? std::min<int64_t>(6, std::max<int64_t>(3, (ku + target - 1) / target))
                                : (int64_t)grp * nkt + 1;
  std::vector<MAttnItem> itf, itk;
  std::vector<MAttnMerge> mf, mk;
  int slots_f = 0, slots_k = 0;
  for (int h = 0; h < nh; h++)
    for (int64_t qb = 0; qb < nlb; qb++)
      attn_cut(fl[(size_t)qb], attn_piece(m, qb), h, (int)qb, 0, (int)t, slots_f, itf, mf);
  for (int g = 0; g < nkv; g++)
    for (int64_t kb = 0; kb < nlb; kb++) attn_cut(kl[(size_t)kb], ck, g, (int)kb, 0, (int)t, slots_k, itk, mk);
  // the merges by (head, 16-row block), for the QK backward that sums the slots itself
  const int64_t nb16 = (t + 15) / 16;
  std::vector<int32_t> qmi((size_t)(nh * nb16), -1), kmi((size_t)(nkv * nb16), -1);
  for (size_t i = 0; i < mf.size(); i++) qmi[(size_t)(mf[i].head * nb16 + mf[i].blk)] = (int32_t)i;
  for (size_t i = 0; i < mk.size(); i++) kmi[(size_t)(mk[i].head * nb16 + mk[i].blk)] = (int32_t)i;
  const auto al = [](size_t b) { return (b + 255) / 256 * 256; };
  const size_t slots = (size_t)slots_f + (size_t)slots_k;  // the dq and dk / dv items run together
  const size_t bytes = al(itf.size() * sizeof(MAttnItem)) + al(itk.size() * sizeof(MAttnItem)) +
                       al(mf.size() * sizeof(MAttnMerge)) + al(mk.size() * sizeof(MAttnMerge)) +
                       al(qmi.size() * 4) + al(kmi.size() * 4) + al(std::max<size_t>(slots, 1) * 32 * (size_t)c.head_dim * 4);
  M_HIP(hipStreamSynchronize(stream_of(m)));
  if (bytes > m->attn_cap) {
    if (m->attn_mem) M_HIP(hipFree(m->attn_mem));
    m->attn_mem = nullptr;
    m->attn_cap = 0;
    M_HIP(hipMalloc(&m->attn_mem, bytes));
    m->attn_cap = bytes;
  }
  char* p = (char*)m->attn_mem;
  m->it_fwd = (MAttnItem*)p;
  p += al(itf.size() * sizeof(MAttnItem));
  m->it_kv = (MAttnItem*)p;
  p += al(itk.size() * sizeof(MAttnItem));
  m->mg_fwd = (MAttnMerge*)p;
  p += al(mf.size() * sizeof(MAttnMerge));
  m->mg_kv = (MAttnMerge*)p;
  p += al(mk.size() * sizeof(MAttnMerge));
  m->qmi = (int32_t*)p;
  p += al(qmi.size() * 4);
  m->kmi = (int32_t*)p;
  p += al(kmi.size() * 4);
  m->attn_part = (float*)p;
  m->attn_part_kv = m->attn_part + (size_t)slots_f * 32 * (size_t)c.head_dim;
  M_HIP(hipMemcpy(m->it_fwd, itf.data(), itf.size() * sizeof(MAttnItem), hipMemcpyHostToDevice));
  M_HIP(hipMemcpy(m->it_kv, itk.data(), itk.size() * sizeof(MAttnItem), hipMemcpyHostToDevice));
  M_HIP(hipMemcpy(m->mg_fwd, mf.data(), mf.size() * sizeof(MAttnMerge), hipMemcpyHostToDevice));
  M_HIP(hipMemcpy(m->mg_kv, mk.data(), mk.size() * sizeof(MAttnMerge), hipMemcpyHostToDevice));
  M_HIP(hipMemcpy(m->qmi, qmi.data(), qmi.size() * 4, hipMemcpyHostToDevice));
  M_HIP(hipMemcpy(m->kmi, kmi.data(), kmi.size() * 4, hipMemcpyHostToDevice));
  m->n_fwd = (int)itf.size();
  m->n_kv = (int)itk.size();
  m->n_mfwd = (int)mf.size();
  m->n_mkv = (int)mk.size();
  m->attn_t = t;
  m->attn_packed = packed;
  m->gen++;
  m->attn_seg.assign(seg ? seg : seg, seg ? seg + t : seg);
  return RTQ_OK;
}

// the packed layout's logical sequences (MSeqArgs) for t tokens of segments seg: for each segment
// value s present, in increasing order, the rows whose segment is 0 or s in packed order, at rows
// [base, base + len) of the gathered buffers (base a multiple of 64); each packed row's own copy
// is the one in its segment's sequence.  With the fused kernels, also the sequences' items: for
// every head and 64-row block of a sequence holding one of its own rows, key tiles 0 .. qb cut by
// attn_piece, exactly the items an unpacked step of that sequence alone would run (its rows at
// rbase = base).  Rebuilt when the segments or the attention path change.
rtq_status ensure_seq_plan(rtq_model* m, int64_t t, const int32_t* seg) {
  if (!seg) {
    m->seq_on = false;
    return RTQ_OK;
  }
  if (m->seq_fused == m->attn_fused && (int64_t)m->seq_seg.size() == t && std::equal(m->seq_seg.begin(), m->seq_seg.end(), seg))
    return RTQ_OK;
  const rtq_model_config& c = m->cfg;
  const int64_t nh = c.n_head, qd = nh * c.head_dim, kd = c.n_head_kv * c.head_dim;
  std::vector<int32_t> vals(seg, seg + t);
  std::sort(vals.begin(), vals.end());
  vals.erase(std::unique(vals.begin(), vals.end()), vals.end());
  int64_t n0 = 0;
  for (int64_t i = 0; i < t; i++) n0 += seg[i] == 0;
  int64_t tv = 0;
  for (int32_t v : vals) {
    int64_t len = n0;
    if (v != 0)
      for (int64_t i = 0; i < t; i++) len += seg[i] == v;
    tv += (len + 63) / 64 * 64;
  }
  m->seq_seg.assign(seg, seg + t);
  m->seq_fused = m->attn_fused;
  m->seqs.clear();
  m->gen++;
  m->seq_on = tv <= 4 * t + 64 * (int64_t)vals.size();
  if (!m->seq_on) return RTQ_OK;
  std::vector<int32_t> gmap, sidx((size_t)t, -1);
  gmap.reserve((size_t)tv);
  for (int32_t v : vals) {
    const int64_t base = (int64_t)gmap.size();
    for (int64_t i = 0; i < t; i++)
      if (seg[i] == 0 || seg[i] == v) {
        if (seg[i] == v) sidx[(size_t)i] = (int32_t)gmap.size();
        gmap.push_back((int32_t)i);
      }
    m->seqs.push_back(rtq_model::SeqRun{base, (int64_t)gmap.size() - base});
    while (gmap.size() % 64) gmap.push_back(-1);
  }
  std::vector<MAttnItem> its;
  std::vector<MAttnMerge> mgs;
  int slots = 0;
  if (m->attn_fused) {
    std::vector<int> L;
    for (int64_t h = 0; h < nh; h++)
      for (size_t q = 0; q < m->seqs.size(); q++) {
        const rtq_model::SeqRun& r = m->seqs[q];
        for (int64_t qb = 0; qb * 64 < r.len; qb++) {
          bool own = false;
          for (int64_t p = qb * 64; p < std::min(r.len, qb * 64 + 64) && !own; p++)
            own = seg[gmap[(size_t)(r.base + p)]] == vals[q];
          if (!own) continue;
          L.resize((size_t)qb + 1);
          for (int64_t kt = 0; kt <= qb; kt++) L[(size_t)kt] = (int)kt;
          attn_cut(L, attn_piece(m, qb), (int)h, (int)qb, (int)r.base, (int)r.len, slots, its, mgs);
        }
      }
  }
  const auto al = [](size_t b) { return (b + 255) / 256 * 256; };
  const size_t bytes = al((size_t)tv * 4) + al((size_t)t * 4) + al(its.size() * sizeof(MAttnItem)) +
                       al(mgs.size() * sizeof(MAttnMerge)) + al((size_t)(tv * qd) * 4) * 2 +
                       al((size_t)(tv * kd) * 4) * 2 + al((size_t)(nh * tv) * 4) +
                       al((size_t)std::max(slots, 1) * 32 * (size_t)c.head_dim * 4);
  M_HIP(hipStreamSynchronize(stream_of(m)));
  if (bytes > m->seq_cap) {
    if (m->seq_mem) M_HIP(hipFree(m->seq_mem));
    m->seq_mem = nullptr;
    m->seq_cap = 0;
    M_HIP(hipMalloc(&m->seq_mem, bytes));
    m->seq_cap = bytes;
  }
  char* p = (char*)m->seq_mem;
  auto take = [&](size_t b) {
    char* q = p;
    p += al(b);
    return q;
  };
  m->gmap_d = (int32_t*)take((size_t)tv * 4);
  m->sidx_d = (int32_t*)take((size_t)t * 4);
  m->it_seq = (MAttnItem*)take(its.size() * sizeof(MAttnItem));
  m->mg_seq = (MAttnMerge*)take(mgs.size() * sizeof(MAttnMerge));
  m->gq = (float*)take((size_t)(tv * qd) * 4);
  m->go = (float*)take((size_t)(tv * qd) * 4);
  m->gk = (float*)take((size_t)(tv * kd) * 4);
  m->gv = (float*)take((size_t)(tv * kd) * 4);
  m->glse = (float*)take((size_t)(nh * tv) * 4);
  m->seq_part = (float*)take((size_t)std::max(slots, 1) * 32 * (size_t)c.head_dim * 4);
  M_HIP(hipMemcpy(m->gmap_d, gmap.data(), gmap.size() * 4, hipMemcpyHostToDevice));
  M_HIP(hipMemcpy(m->sidx_d, sidx.data(), sidx.size() * 4, hipMemcpyHostToDevice));
  if (!its.empty()) M_HIP(hipMemcpy(m->it_seq, its.data(), its.size() * sizeof(MAttnItem), hipMemcpyHostToDevice));
  if (!mgs.empty()) M_HIP(hipMemcpy(m->mg_seq, mgs.data(), mgs.size() * sizeof(MAttnMerge), hipMemcpyHostToDevice));
  m->tv = tv;
  m->n_sit = (int)its.size();
  m->n_smg = (int)mgs.size();
  return RTQ_OK;
}

MAttnArgs attn_args(rtq_model* m, Cache& k, int64_t t) {
  const rtq_model_config& c = m->cfg;
  MAttnArgs a{};
  a.q = k.q;
  a.k = k.k;
  a.v = k.v;
  a.o = k.o;
  a.lse = k.lse;
  a.D = m->attn_D;
  a.part = m->attn_part;
  a.seg = m->packed ? m->seg_d : nullptr;
  a.live = m->packed ? m->live_d : nullptr;
  a.nlb = (int)m->nlb;
  a.t = (int)t;
  a.nh = (int)c.n_head;
  a.nkv = (int)c.n_head_kv;
  a.hd = (int)c.head_dim;
  a.ldq = c.n_head * c.head_dim;
  a.ldk = a.ldv = c.n_head_kv * c.head_dim;
  a.scale = 1.0f / sqrtf((float)c.head_dim);
  const int64_t qd = c.n_head * c.head_dim, kd = c.n_head_kv * c.head_dim, tp = (t + 63) / 64 * 64;
  a.tp = (int)tp;
  if (m->attn_fused) {  // planes for t tokens laid out back to back (the buffer holds t_cap)
    uint16_t* p = m->attn_planes;
    for (uint16_t** q : {&a.pqsh, &a.pqsl, &a.pdoh, &a.pdol}) *q = p, p += t * qd;
    a.pkf = p, p += t * kd;
    a.pvh = p, p += t * kd;
    a.pvl = p, p += t * kd;
    for (uint16_t** q : {&a.pqth, &a.pqtl, &a.pdth, &a.pdtl}) *q = p, p += tp * qd;
    a.pkth = p, p += tp * kd;
    a.pktl = p;
  }
  return a;
}

// launches an item pass (one wave per item, four per workgroup)
// one workgroup (four waves) per item
rtq_status attn_launch(rtq_model* m, int km, MAttnArgs a, const MAttnItem* items, int n) {
  if (n <= 0) return RTQ_OK;
  a.items = items;
  a.n_items = n;
  return rtq_model_launch(m->ctx, km, dim3((unsigned)n), dim3(256), stream_of(m), &a);
}
// one thread per element of each merged block (16 x hd)
rtq_status attn_merge(rtq_model* m, int km, MAttnArgs a, const MAttnMerge* mg, int n) {
  if (n <= 0) return RTQ_OK;
  a.merges = mg;
  a.n_merges = n;
  const int64_t nel4 = 4 * (int64_t)a.hd;  // threads per 16 x hd block: four elements each
  return rtq_model_launch(m->ctx, km, dim3((unsigned)(n * ((nel4 + 255) / 256))), dim3(256), stream_of(m), &a);
}

// ---------------------------------------------------------------- one block
// q, k, v raw rows in a cache's qkv buffer (or the gradient buffer of the same layout)
struct QkvView {
  float *q, *k, *v;
  int64_t ldq, ldk, ldv;
};

QkvView qkv_view(const rtq_model* m, const Layer& L, float* base, int64_t t) {
  const rtq_model_config& c = m->cfg;
  const int64_t qd = c.n_head * c.head_dim, kd = c.n_head_kv * c.head_dim;
  if (L.qkv_fused) return QkvView{base, base + qd, base + qd + kd, qd + 2 * kd, qd + 2 * kd, qd + 2 * kd};
  return QkvView{base, base + t * qd, base + t * (qd + kd), qd, kd, kd};
}

// a block's gradient buffers: its own (deferred dA / dB) or the step-wide ones
float* g_dqkv(rtq_model* m, const Cache& k) { return k.dqkv ? k.dqkv : m->dqkv; }
float* g_dgu(rtq_model* m, const Cache& k) { return k.dgu ? k.dgu : m->dgu; }
float* g_dh(rtq_model* m, const Cache& k) { return k.dh ? k.dh : m->dh; }

// the deferred dA / dB of the whole step in one launch: the job table and its workgroup map
// (job, tile) are uploaded to device memory when the jobs differ from the last upload (a new
// shape; a captured or replayed step reuses the table)
rtq_status lora_grads_all(rtq_model* m) {
  std::vector<LoraGradArgs> jobs;
  std::vector<int> map;
  std::vector<uintptr_t> key;
  int64_t tmax = 0;
  for (const LoraGradArgs& j : m->lg_all) {
    const int n = j.n_gb + j.n_ga;
    if (n == 0) continue;
    const int ji = (int)jobs.size();
    jobs.push_back(j);
    // tile b = row tile * jt + rank tile: the jt rank tiles of a row tile (which read the same dy or
    // x rows) placed 8 workgroups apart, so that they run on one XCD and share its L2 (workgroups
    // go to the 8 XCDs in turn): per section (gb, then ga), blocks of 8 row tiles, rank tile by
    // rank tile.  Each tile writes its own outputs: the order changes no result.
    const int jt = (j.r + 15) / 16;
    for (int sec = 0; sec < 2; sec++) {
      const int b0 = sec ? j.n_gb : 0, nrt = (sec ? j.n_ga : j.n_gb) / std::max(jt, 1);
      for (int r0 = 0; r0 < nrt; r0 += 8)
        for (int jj = 0; jj < jt; jj++)
          for (int rt = r0; rt < std::min(r0 + 8, nrt); rt++) {
            map.push_back(ji);
            map.push_back(b0 + rt * jt + jj);
          }
    }
    tmax = std::max<int64_t>(tmax, j.T);
    for (uintptr_t v : {(uintptr_t)j.dy, (uintptr_t)j.h, (uintptr_t)j.g, (uintptr_t)j.x, (uintptr_t)j.la,
                        (uintptr_t)j.gb, (uintptr_t)j.ga, (uintptr_t)j.T, (uintptr_t)j.N, (uintptr_t)j.K,
                        (uintptr_t)j.r, (uintptr_t)j.n_gb, (uintptr_t)j.n_ga, (uintptr_t)__builtin_bit_cast(uint32_t, j.s)})
      key.push_back(v);
  }
  m->lg_all.clear();
  if (jobs.empty()) return RTQ_OK;
  const size_t jb = (jobs.size() * sizeof(LoraGradArgs) + 255) / 256 * 256, bytes = jb + map.size() * sizeof(int);
  hipStream_t st = stream_of(m);
  if (bytes > m->lgt_cap) {
    M_HIP(hipStreamSynchronize(st));
    if (m->lgt_mem) M_HIP(hipFree(m->lgt_mem));
    if (m->lgt_host) M_HIP(hipHostFree(m->lgt_host));
    m->lgt_mem = m->lgt_host = nullptr;
    m->lgt_cap = 0;
    M_HIP(hipMalloc(&m->lgt_mem, bytes));
    M_HIP(hipHostMalloc(&m->lgt_host, bytes));
    m->lgt_cap = bytes;
    m->gen++;
    m->lgt_key.clear();
  }
  if (key != m->lgt_key) {
    M_HIP(hipStreamSynchronize(st));  // an earlier upload may still read the staging buffer
    std::memcpy(m->lgt_host, jobs.data(), jobs.size() * sizeof(LoraGradArgs));
    std::memcpy((char*)m->lgt_host + jb, map.data(), map.size() * sizeof(int));
    M_HIP(hipMemcpyAsync(m->lgt_mem, m->lgt_host, bytes, hipMemcpyHostToDevice, st));
    m->lgt_key = key;
  }
  // 16-wave workgroups from 1024 tokens: below that the whole step's tiles fill the chip with
  // 4-wave ones, each wave looping over more tokens (512 tokens: 0.43 against 0.51 ms; one
  // block's batch, with 16 times fewer tiles, keeps 16 waves from 256 tokens)
  return rtq_lora_grads_table_d(m->ctx, (const LoraGradArgs*)m->lgt_mem, (const int*)((char*)m->lgt_mem + jb),
                                (int64_t)(map.size() / 2), tmax >= 1024, st);
}

// the QK kernels' half-wave rows: head size and rotary width 128 (16-byte aligned rows follow)
bool qk_half(const rtq_model* m) { return m->cfg.head_dim == 128 && m->cfg.rope_dim == 128; }
// workgroups of the QK kernels for `rows` (token, head) rows: 8 per workgroup (half-wave rows) or 4
unsigned qk_grid(const rtq_model* m, int64_t rows) { return (unsigned)(qk_half(m) ? (rows + 7) / 8 : (rows + 3) / 4); }

MQkArgs qk_args(rtq_model* m, const Layer& L, Cache& k, int64_t t) {
  const rtq_model_config& c = m->cfg;
  const QkvView x = qkv_view(m, L, k.qkv, t), dx = qkv_view(m, L, g_dqkv(m, k), t);
  return MQkArgs{x.q,   x.k,   x.v,   L.q_norm, L.k_norm, m->cos_,          m->sin_,          k.q,
                 k.k,   k.v,   k.q_inv, k.k_inv, m->dq,     m->dk,            dx.q,             dx.k,
                 (int)t, (int)c.n_head, (int)c.n_head_kv, (int)c.head_dim, (int)c.rope_dim, c.rope_neox,
                 c.kv_f16, c.rms_eps, c.norm_offset, x.ldq, x.ldk, x.ldv, qk_half(m) ? 1 : 0};
}

// gate | u views of a cache's gu buffer (or the gradient buffer of the same layout)
void gu_view(const rtq_model* m, const Layer& L, float* base, int64_t t, float** g, float** u, int64_t* ld) {
  const int64_t ff = m->cfg.n_ff;
  *g = base;
  *u = L.gu_fused ? base + ff : base + t * ff;
  *ld = L.gu_fused ? 2 * ff : ff;
}

// add_in: x is not written yet: it is the previous block's output h + mlp (its h in its cache, mlp
// in f), summed by this block's first norm kernel (which writes x); add_out: this block writes y,
// else it leaves h (cache) and mlp (f) for the next block's first norm
rtq_status block_forward(rtq_model* m, int l, int64_t t, float* x, float* y, bool add_in, bool add_out) {
  const rtq_model_config& c = m->cfg;
  const Layer& L = m->layers[(size_t)l];
  Cache& k = m->cache[m->ckpt ? 0 : (size_t)l];
  const int64_t d = c.n_embd, nh = c.n_head, nkv = c.n_head_kv, hd = c.head_dim, grp = nh / nkv;
  const int64_t qd = nh * hd, kd = nkv * hd;
  // x = h + mlp of block l - 1 (src/model.rs:196), n1 = rmsnorm(x)
  const float* in_a = add_in ? m->cache[m->ckpt ? 0 : (size_t)(l - 1)].h : x;
  const float* in_b = add_in ? m->f : nullptr;
  float* in_h = add_in ? x : nullptr;
  const QkvView qv = qkv_view(m, L, k.qkv, t);
  if (L.qkv_fused) {
    M_TRY(lin_fwd_norm(m, L.groups[(size_t)L.gi[LQ]], in_a, in_b, in_h, L.attn_norm, k.n1, k.inv1, t, k.qkv));
  } else {
    M_TRY(lin_fwd_norm(m, L.groups[(size_t)L.gi[LQ]], in_a, in_b, in_h, L.attn_norm, k.n1, k.inv1, t, qv.q));
    M_TRY(lin_fwd(m, L.groups[(size_t)L.gi[LK]], k.n1, t, qv.k));
    M_TRY(lin_fwd(m, L.groups[(size_t)L.gi[LV]], k.n1, t, qv.v));
  }
  const MQkArgs qa = qk_args(m, L, k, t);
  M_TRY(rtq_model_launch(m->ctx, KM_QK_PREP, dim3(qk_grid(m, t * (nh + 2 * nkv))), dim3(256), stream_of(m),
                         &qa));
  const float scale = 1.0f / sqrtf((float)hd);
  // a packed layout's forward runs over each segment's logical sequence (ensure_seq_plan): every
  // row gets the bits of its example's own unpacked step
  const bool seq = m->packed && m->seq_on;
  const MSeqArgs sq{k.q, k.k, k.v, m->gq, m->gk, m->gv, m->go, m->attn_fused ? m->glse : nullptr, k.o, k.lse,
                    m->gmap_d, m->sidx_d, (int)t, (int)m->tv, (int)nh, (int)nkv, (int)hd, qd, kd, kd};
  if (seq)
    M_TRY(rtq_model_launch(m->ctx, KM_SEQ_GATHER, dim3((unsigned)m->tv), dim3(256), stream_of(m), &sq));
  if (m->attn_fused && seq) {
    MAttnArgs aa = attn_args(m, k, t);
    aa.q = m->gq, aa.k = m->gk, aa.v = m->gv, aa.o = m->go, aa.lse = m->glse, aa.part = m->seq_part;
    aa.seg = nullptr, aa.live = nullptr, aa.nlb = 0, aa.t = (int)m->tv;
    M_TRY(attn_launch(m, hd == 64 ? KM_FA_FWD64 : KM_FA_FWD128, aa, m->it_seq, m->n_sit));
    M_TRY(attn_merge(m, KM_ATTN_MERGE_FWD, aa, m->mg_seq, m->n_smg));
  } else if (m->attn_fused) {  // fused: o and each row's log-sum-exp, no probability matrix
    const MAttnArgs aa = attn_args(m, k, t);
    M_TRY(attn_launch(m, hd == 64 ? KM_FA_FWD64 : KM_FA_FWD128, aa, m->it_fwd, m->n_fwd));
    M_TRY(attn_merge(m, KM_ATTN_MERGE_FWD, aa, m->mg_fwd, m->n_mfwd));
  } else {
  if (seq) {  // each sequence as an unpacked step of its own length (dP holds its probabilities)
    m->seq_pass = true;
    for (const rtq_model::SeqRun& r : m->seqs) {
      const int64_t n = r.len;
      const float *gq = m->gq + r.base * qd, *gk = m->gk + r.base * kd, *gv = m->gv + r.base * kd;
      M_TRY(k_gemm(m, n, n, hd, nh, Op{gq, hd, qd, 1, 1}, Op{gk, hd, 1, kd, (int)grp}, m->dP, n * n, n, 1, scale, 1,
                   0, SPLIT_HF));
      MSoftArgs ss{m->dP, nullptr, nullptr, (int)n, (int)nh, scale, nullptr, nullptr, 0};
      M_TRY(rtq_model_launch(m->ctx, KM_SOFTMAX, dim3((unsigned)((n + 3) / 4), (unsigned)nh), dim3(256),
                             stream_of(m), &ss));
      M_TRY(k_gemm(m, n, hd, n, nh, Op{m->dP, n * n, n, 1, 1}, Op{gv, hd, kd, 1, (int)grp}, m->go + r.base * qd, hd,
                   qd, 1, 1.0f, 2, 0, SPLIT_HF));
    }
    m->seq_pass = false;
  }
  // S = (q scale) K^T per head (causal), softmax in place, O = P V (a packed layout's P, for the
  // backward, over the packed rows)
  M_TRY(k_gemm(m, t, t, hd, nh, Op{k.q, hd, qd, 1, 1}, Op{k.k, hd, 1, kd, (int)grp}, k.P, t * t, t, 1, scale, 1, 0,
               SPLIT_HF));
  MSoftArgs sa{k.P, nullptr, nullptr, (int)t, (int)nh, scale, m->packed ? m->seg_d : nullptr,
               m->packed ? m->live_d : nullptr, (int)m->nlb};
  M_TRY(rtq_model_launch(m->ctx, KM_SOFTMAX, dim3((unsigned)((t + 3) / 4), (unsigned)nh), dim3(256), stream_of(m),
                         &sa));
  if (!seq)
    M_TRY(k_gemm(m, t, hd, t, nh, Op{k.P, t * t, t, 1, 1}, Op{k.v, hd, kd, 1, (int)grp}, k.o, hd, qd, 1, 1.0f, 2, 0,
                 SPLIT_HF));
  }
  if (seq) M_TRY(rtq_model_launch(m->ctx, KM_SEQ_SCATTER, dim3((unsigned)t), dim3(256), stream_of(m), &sq));
  M_TRY(lin_fwd(m, L.groups[(size_t)L.gi[LO]], k.o, t, m->mo));
  float *g, *u;
  int64_t ldg;
  gu_view(m, L, k.gu, t, &g, &u, &ldg);
  // h = x + attn, n2 = rmsnorm(h)
  if (L.gu_fused) {
    M_TRY(lin_fwd_norm(m, L.groups[(size_t)L.gi[LGATE]], x, m->mo, k.h, L.ffn_norm, k.n2, k.inv2, t, k.gu));
  } else {
    M_TRY(lin_fwd_norm(m, L.groups[(size_t)L.gi[LGATE]], x, m->mo, k.h, L.ffn_norm, k.n2, k.inv2, t, g));
    M_TRY(lin_fwd(m, L.groups[(size_t)L.gi[LUP]], k.n2, t, u));
  }
  M_TRY(lin_fwd_swiglu(m, L.groups[(size_t)L.gi[LDOWN]], g, u, ldg, k.hm, t, m->f));
  if (!add_out) return RTQ_OK;
  return k_elt(m, KM_ADD, k.h, m->f, nullptr, y, nullptr, t * d);  // y = h + mlp
}

rtq_status block_backward(rtq_model* m, int l, int64_t t, const float* x, const float* dy, float* dx) {
  const rtq_model_config& c = m->cfg;
  const Layer& L = m->layers[(size_t)l];
  Cache& k = m->cache[m->ckpt ? 0 : (size_t)l];
  const int64_t d = c.n_embd, nh = c.n_head, nkv = c.n_head_kv, hd = c.head_dim, grp = nh / nkv;
  const int64_t qd = nh * hd, kd = nkv * hd;
  const float scale = 1.0f / sqrtf((float)hd);
  // Mlp::backward (src/model.rs:120-133)
  std::vector<LoraGradArgs> jobs;  // this block's dA / dB: launched before its last kernel, or deferred
  float* const dgu = g_dgu(m, k);
  float* const dqkv = g_dqkv(m, k);
  float* const dh = g_dh(m, k);
  float *g, *u, *dg, *du;
  int64_t ldg;
  gu_view(m, L, k.gu, t, &g, &u, &ldg);
  gu_view(m, L, dgu, t, &dg, &du, &ldg);
  // dhm's SwiGLU backward in the down projection's dx finish (dhm itself kept for a captured layer)
  const SwiGluBwd sw{g, u, dg, du, ldg, l == m->dbg_layer};
  bool sw_done = false;
  M_TRY(lin_bwd(m, L, L.gi[LDOWN], k.hm, dy, t, m->dhm, &jobs, &sw, &sw_done));
  if (!sw_done) M_TRY(k_elt2(m, KM_SWIGLU_BWD, g, u, m->dhm, dg, du, t, c.n_ff, ldg, c.n_ff, ldg));
  if (L.gu_fused) {
    M_TRY(lin_bwd(m, L, L.gi[LGATE], k.n2, dgu, t, m->dn2, &jobs));  // dgate.Wg + dup.Wu in one pass
  } else {
    M_TRY(lin_bwd(m, L, L.gi[LGATE], k.n2, dg, t, m->dn2, &jobs));
    M_TRY(lin_bwd(m, L, L.gi[LUP], k.n2, du, t, m->dxu, &jobs));
    M_TRY(k_elt(m, KM_ADD, m->dn2, m->dxu, nullptr, m->dn2, nullptr, t * d));
  }
  M_TRY(k_norm_bwd(m, k.h, L.ffn_norm, k.inv2, m->dn2, dy, dh, t, d));  // dh = dy + rmsnorm_backward
  // Attention::backward (src/attention.rs:243-355)
  M_TRY(lin_bwd(m, L, L.gi[LO], k.o, dh, t, m->d_o, &jobs));
  const QkvView dv = qkv_view(m, L, dqkv, t);
  if (m->attn_fused) {  // D = dO . o; dq over key tiles; dk, dv over (group head, query tile) pairs
    MAttnArgs aa = attn_args(m, k, t);
    aa.dO = m->d_o;
    aa.dq = m->dq;
    aa.dk = m->dk;
    aa.dv = dv.v;
    aa.ld_dv = dv.ldv;
    // D and the 16-bit operand planes of q, dO, k, v, once per layer
    M_TRY(rtq_model_launch(m->ctx, hd == 64 ? KM_ATTN_BWD_PREP64 : KM_ATTN_BWD_PREP128,
                           dim3((unsigned)((t + 63) / 64 * 4), (unsigned)(nh + nkv)), dim3(256), stream_of(m), &aa));
    aa.items = m->it_fwd;  // dq over key tiles, and dk, dv over (group head, query tile) pairs: one launch
    aa.n_items = m->n_fwd;
    aa.items2 = m->it_kv;
    aa.n_items2 = m->n_kv;
    aa.part2 = m->attn_part_kv;
    M_TRY(rtq_model_launch(m->ctx, hd == 64 ? KM_FA_BWD64 : KM_FA_BWD128, dim3((unsigned)(m->n_fwd + m->n_kv)),
                           dim3(256), stream_of(m), &aa));
    aa.merges = m->mg_fwd;
    aa.n_merges = m->n_mfwd;
    aa.merges2 = m->mg_kv;
    aa.n_merges2 = m->n_mkv;
    const int64_t nmb = m->n_mkv * ((8 * hd + 255) / 256) + m->n_mfwd * ((4 * hd + 255) / 256);
    // the QK backward's half-wave rows sum the slots of cut blocks themselves (a captured layer
    // keeps the merge launch, so that its dq, dk are whole)
    if (nmb > 0 && !(qk_half(m) && l != m->dbg_layer))
      M_TRY(rtq_model_launch(m->ctx, KM_ATTN_MERGE_BWD, dim3((unsigned)nmb), dim3(256), stream_of(m), &aa));
  } else {
  M_TRY(k_gemm(m, t, t, hd, nh, Op{m->d_o, hd, qd, 1, 1}, Op{k.v, hd, 1, kd, (int)grp}, m->dP, t * t, t, 1, 1.0f, 1,
               0, SPLIT_BF));  // dP = dO V^T
  MSoftArgs sa{nullptr, k.P, m->dP, (int)t, (int)nh, scale, m->packed ? m->seg_d : nullptr,
               m->packed ? m->live_d : nullptr, (int)m->nlb};
  M_TRY(rtq_model_launch(m->ctx, KM_SOFTMAX_BWD, dim3((unsigned)((t + 3) / 4), (unsigned)nh), dim3(256),
                         stream_of(m), &sa));
  // dV_h = P^T dO, dQ = dS K, dK_h = dS^T Q: independent, one launch
  const GemmJob jobs[3] = {
      {t, hd, t, nh, Op{k.P, t * t, 1, t, 1}, Op{m->d_o, hd, qd, 1, 1}, m->dvh, t * hd, hd, 1, 1.0f, 3, 0},
      {t, hd, t, nh, Op{m->dP, t * t, t, 1, 1}, Op{k.k, hd, kd, 1, (int)grp}, m->dq, hd, qd, 1, 1.0f, 2, 0},
      {t, hd, t, nh, Op{m->dP, t * t, 1, t, 1}, Op{k.q, hd, qd, 1, 1}, m->dkh, t * hd, hd, 1, 1.0f, 3, 0}};
  M_TRY(k_gemm_group(m, jobs, 3));
  MGroupArgs gsa{m->dkh, m->dvh, m->dk, dv.v, (int)t, (int)nh, (int)nkv, (int)hd, dv.ldv};
  M_TRY(rtq_model_launch(m->ctx, KM_GROUP_SUM, dim3((unsigned)std::min<int64_t>((t * kd + 255) / 256, 4096)),
                         dim3(256), stream_of(m), &gsa));
  }
  MQkArgs qa = qk_args(m, L, k, t);
  if (m->attn_fused && qk_half(m) && l != m->dbg_layer) {
    qa.qmi = m->qmi;
    qa.kmi = m->kmi;
    qa.qmerges = m->mg_fwd;
    qa.kmerges = m->mg_kv;
    qa.qpart = m->attn_part;
    qa.kpart = m->attn_part_kv;
    qa.dv = dv.v;
    qa.ld_dv = dv.ldv;
    qa.nb16 = (int)((t + 15) / 16);
  }
  M_TRY(rtq_model_launch(m->ctx, KM_QK_BWD, dim3(qk_grid(m, t * (nh + nkv))), dim3(256), stream_of(m), &qa));
  if (L.qkv_fused) {
    M_TRY(lin_bwd(m, L, L.gi[LQ], k.n1, dqkv, t, m->dn1, &jobs));  // dq.Wq + dk.Wk + dv.Wv in one pass
  } else {
    M_TRY(lin_bwd(m, L, L.gi[LQ], k.n1, dv.q, t, m->dn1, &jobs));
    M_TRY(lin_bwd(m, L, L.gi[LK], k.n1, dv.k, t, m->dxk, &jobs));
    M_TRY(lin_bwd(m, L, L.gi[LV], k.n1, dv.v, t, m->dxv, &jobs));
    M_TRY(k_elt(m, KM_ADD, m->dn1, m->dxk, m->dxv, m->dn1, nullptr, t * d));  // dq + (dk + dv)
  }
  // every input of the deferred dA / dB (dy, x of each linear, the h / g slots) is still intact here.
  // (Run on a second stream, overlapping the next block's backward, the batch measured slower:
  // 13.79 against 13.45 ms per configs[2] step - its workgroups hold CUs the next dx kernels need.)
  if (m->defer_lg)  // every input (dy, x of each linear, the layer's h / g slots) stays intact to the end
    m->lg_all.insert(m->lg_all.end(), jobs.begin(), jobs.end());
  else
    M_TRY(rtq_lora_grads_d(m->ctx, jobs.data(), (int)jobs.size(), stream_of(m)));
  return k_norm_bwd(m, x, L.attn_norm, k.inv1, m->dn1, dh, dx, t, d);  // dx = dh + rmsnorm_backward
}

// ---------------------------------------------------------------- debug capture
// rtq_model_debug_capture: copies of one layer's tensors taken during the step, in plain row-major
// layouts (per token: q_raw [qd], k_raw / v_raw [kd], gate / up [ff], ...)
rtq_status dbg_put(rtq_model* m, const char* name, const float* src, int64_t rows, int64_t cols, int64_t ld) {
  float* dst = nullptr;
  for (auto& e : m->dbg)
    if (e.first == name) {
      if (e.second.second != rows * cols) {
        dev_free(m, e.second.first);
        e.second.first = nullptr;
      }
      dst = e.second.first;
      if (!dst) {
        void* p;
        M_TRY(dev_alloc(m, (size_t)(rows * cols) * 4, &p));
        e.second = {(float*)p, rows * cols};
        dst = (float*)p;
      }
    }
  if (!dst) {
    void* p;
    M_TRY(dev_alloc(m, (size_t)(rows * cols) * 4, &p));
    m->dbg.push_back({name, {(float*)p, rows * cols}});
    dst = (float*)p;
  }
  M_HIP(hipMemcpy2DAsync(dst, (size_t)cols * 4, src, (size_t)ld * 4, (size_t)cols * 4, (size_t)rows,
                         hipMemcpyDeviceToDevice, stream_of(m)));
  return RTQ_OK;
}

rtq_status dbg_forward(rtq_model* m, int l, int64_t t, const float* x, const float* y) {
  const rtq_model_config& c = m->cfg;
  const Layer& L = m->layers[(size_t)l];
  Cache& k = m->cache[m->ckpt ? 0 : (size_t)l];
  const int64_t d = c.n_embd, qd = c.n_head * c.head_dim, kd = c.n_head_kv * c.head_dim, ff = c.n_ff;
  const QkvView qv = qkv_view(m, L, k.qkv, t);
  float *g, *u;
  int64_t ldg;
  gu_view(m, L, k.gu, t, &g, &u, &ldg);
  M_TRY(dbg_put(m, "x", x, t, d, d));
  M_TRY(dbg_put(m, "n1", k.n1, t, d, d));
  M_TRY(dbg_put(m, "inv1", k.inv1, 1, t, t));
  M_TRY(dbg_put(m, "q_raw", qv.q, t, qd, qv.ldq));
  M_TRY(dbg_put(m, "k_raw", qv.k, t, kd, qv.ldk));
  M_TRY(dbg_put(m, "v_raw", qv.v, t, kd, qv.ldv));
  M_TRY(dbg_put(m, "q", k.q, t, qd, qd));
  M_TRY(dbg_put(m, "k", k.k, t, kd, kd));
  M_TRY(dbg_put(m, "v", k.v, t, kd, kd));
  M_TRY(dbg_put(m, "q_inv", k.q_inv, 1, t * c.n_head, t * c.n_head));
  M_TRY(dbg_put(m, "k_inv", k.k_inv, 1, t * c.n_head_kv, t * c.n_head_kv));
  if (m->attn_fused) M_TRY(dbg_put(m, "lse", k.lse, c.n_head, t, t));
  else M_TRY(dbg_put(m, "P", k.P, c.n_head * t, t, t));
  M_TRY(dbg_put(m, "o", k.o, t, qd, qd));
  M_TRY(dbg_put(m, "h", k.h, t, d, d));
  M_TRY(dbg_put(m, "n2", k.n2, t, d, d));
  M_TRY(dbg_put(m, "inv2", k.inv2, 1, t, t));
  M_TRY(dbg_put(m, "gate", g, t, ff, ldg));
  M_TRY(dbg_put(m, "up", u, t, ff, ldg));
  M_TRY(dbg_put(m, "hm", k.hm, t, ff, ff));
  return dbg_put(m, "y", y, t, d, d);
}

rtq_status dbg_backward(rtq_model* m, int l, int64_t t, const float* dy, const float* dx) {
  const rtq_model_config& c = m->cfg;
  const Layer& L = m->layers[(size_t)l];
  const int64_t d = c.n_embd, qd = c.n_head * c.head_dim, kd = c.n_head_kv * c.head_dim, ff = c.n_ff;
  Cache& k = m->cache[m->ckpt ? 0 : (size_t)l];
  const QkvView dv = qkv_view(m, L, g_dqkv(m, k), t);
  float *dg, *du;
  int64_t ldg;
  gu_view(m, L, g_dgu(m, k), t, &dg, &du, &ldg);
  M_TRY(dbg_put(m, "dy", dy, t, d, d));
  M_TRY(dbg_put(m, "dhm", m->dhm, t, ff, ff));
  M_TRY(dbg_put(m, "dgate", dg, t, ff, ldg));
  M_TRY(dbg_put(m, "dup", du, t, ff, ldg));
  M_TRY(dbg_put(m, "dn2", m->dn2, t, d, d));
  M_TRY(dbg_put(m, "dh", g_dh(m, k), t, d, d));
  M_TRY(dbg_put(m, "d_o", m->d_o, t, qd, qd));
  if (!m->attn_fused) M_TRY(dbg_put(m, "dS", m->dP, c.n_head * t, t, t));
  M_TRY(dbg_put(m, "dq", m->dq, t, qd, qd));
  M_TRY(dbg_put(m, "dk", m->dk, t, kd, kd));
  M_TRY(dbg_put(m, "dv", dv.v, t, kd, dv.ldv));
  M_TRY(dbg_put(m, "dq_raw", dv.q, t, qd, dv.ldq));
  M_TRY(dbg_put(m, "dk_raw", dv.k, t, kd, dv.ldk));
  M_TRY(dbg_put(m, "dn1", m->dn1, t, d, d));
  return dbg_put(m, "dx", dx, t, d, d);
}

// the ggml type, packed bytes and shape of a GGUF tensor
rtq_status tensor_bytes(const rtq_gguf* g, const std::string& name, int* type, const uint8_t** data, size_t* nbytes) {
  const int64_t i = rtq_gguf_find_tensor(g, name.c_str());
  if (i < 0) return rtq_fail(RTQ_ERR_INVALID, "GGUF: missing tensor %s", name.c_str());
  const void* d = nullptr;
  M_TRY(rtq_gguf_tensor(g, i, nullptr, type, nullptr, nullptr, &d, nbytes));
  *data = (const uint8_t*)d;
  return RTQ_OK;
}

// the layer's linears as groups: q | k | v and gate | up fused when their ggml types agree
rtq_status load_groups(rtq_model* m, const rtq_gguf* g, const std::string& p, Layer& L, const int64_t* outs,
                       const int64_t* ins) {
  const int sets[4][3] = {{LQ, LK, LV}, {LO, -1, -1}, {LGATE, LUP, -1}, {LDOWN, -1, -1}};
  for (const auto& set : sets) {
    int n = 0, type0 = -1;
    bool same = true;
    for (int j = 0; j < 3 && set[j] >= 0; j++, n++) {
      int type = 0;
      const uint8_t* d;
      size_t nb;
      M_TRY(tensor_bytes(g, p + kLinName[set[j]] + ".weight", &type, &d, &nb));
      same = same && (j == 0 || type == type0);
      type0 = j == 0 ? type : type0;
    }
    const int parts = same ? 1 : n;  // one fused group, or one group per linear
    for (int q = 0; q < parts; q++) {
      Group G;
      const int first = same ? 0 : q, last = same ? n : q + 1;
      std::vector<uint8_t> bytes;
      std::vector<float> bias;
      bool any_bias = false;
      int type = 0;
      for (int j = first; j < last; j++) {
        const int li = set[j];
        const uint8_t* d;
        size_t nb;
        M_TRY(tensor_bytes(g, p + kLinName[li] + ".weight", &type, &d, &nb));
        Member& mb = G.mem[G.nm++];
        mb.lin = li;
        mb.row0 = G.rows;
        mb.rows = outs[li];
        G.rows += outs[li];
        G.in = ins[li];
        L.gi[li] = (int)L.groups.size();
        L.mi[li] = G.nm - 1;
        if (last - first == 1) {  // a lone linear uploads straight from the image
          M_TRY(load_weight(m, g, p + kLinName[li] + ".weight", outs[li], ins[li], &G.w));
        } else {
          bytes.insert(bytes.end(), d, d + nb);
        }
        const int64_t bi = li <= LV ? rtq_gguf_find_tensor(g, (p + kLinName[li] + ".bias").c_str()) : -1;
        std::vector<float> b((size_t)outs[li], 0.0f);
        if (bi >= 0) {
          const void* bd;
          size_t bn;
          int bt = 0;
          M_TRY(rtq_gguf_tensor(g, bi, nullptr, &bt, nullptr, nullptr, &bd, &bn));
          if (bt != RTQ_TYPE_F32 || bn != (size_t)outs[li] * 4)
            return rtq_fail(RTQ_ERR_UNSUPPORTED, "GGUF: %s.bias must be F32", (p + kLinName[li]).c_str());
          memcpy(b.data(), bd, bn);
          any_bias = true;
        }
        bias.insert(bias.end(), b.begin(), b.end());
      }
      if (!G.w) {
        M_TRY(rtq_weight_create(m->ctx, type, bytes.data(), bytes.size(), G.rows, G.in, &G.w));
        m->weights.push_back(G.w);
      }
      if (any_bias) {  // absent biases are zeros: y + 0 = y
        void* bd;
        M_TRY(dev_alloc(m, bias.size() * 4, &bd));
        M_HIP(hipMemcpy(bd, bias.data(), bias.size() * 4, hipMemcpyHostToDevice));
        G.bias = (const float*)bd;
      }
      L.groups.push_back(G);
    }
    if (set[0] == LQ) L.qkv_fused = same;
    if (set[0] == LGATE) L.gu_fused = same;
  }
  return RTQ_OK;
}

}  // namespace

extern "C" {

}  // extern "C"

namespace {
// hyper-parameters and the loader's refusals (load_gguf_from, src/rie.rs:164-260), no device work;
// factors: rope_freqs.weight (or null)
rtq_status parse_config(const rtq_gguf* g, rtq_model_config* out, std::vector<float>* factors) {
  const char* arch_p = nullptr;
  uint64_t arch_n = 0;
  M_TRY(rtq_gguf_get_str(g, "general.architecture", &arch_p, &arch_n));
  const std::string arch(arch_p, arch_n);
  // trainable_arch (src/rie.rs:153-155, :170-172): the decoders whose forward the step reproduces
  // (Mistral GGUFs declare "llama")
  if (arch != "llama" && arch != "qwen2" && arch != "qwen3")
    return rtq_fail(RTQ_ERR_UNSUPPORTED,
                    "architecture '%s' is not trainable yet (supported: llama, mistral, qwen2, qwen3)", arch.c_str());
  rtq_model_config c{};
  c.n_layer = (int64_t)kv_num(g, arch + ".block_count", 0);
  c.n_embd = (int64_t)kv_num(g, arch + ".embedding_length", 0);
  c.n_head = (int64_t)kv_num(g, arch + ".attention.head_count", 0);
  c.n_head_kv = (int64_t)kv_num(g, arch + ".attention.head_count_kv", (double)c.n_head);
  c.head_dim = (int64_t)kv_num(g, arch + ".attention.key_length", c.n_head ? (double)(c.n_embd / c.n_head) : 0);
  c.rope_dim = (int64_t)kv_num(g, arch + ".rope.dimension_count", (double)c.head_dim);
  c.n_ff = (int64_t)kv_num(g, arch + ".feed_forward_length", 0);
  c.rms_eps = (float)kv_num(g, arch + ".attention.layer_norm_rms_epsilon", 1e-6);
  c.rope_base = (float)kv_num(g, arch + ".rope.freq_base", 10000.0);
  c.rope_freq_scale = 1.0f;
  c.norm_offset = 0.0f;
  // the loader's "plain" model check (src/rie.rs:173-183: embedding / residual / logit scale 1, no
  // softcaps, no sliding window, attention scale 1/sqrt(head_dim)) and its dense-FFN check
  // (:211-216), on the GGUF keys that carry those settings
  auto kv_is = [&](const char* key, double plain) {
    double v = 0.0;
    return rtq_gguf_get_f64(g, (arch + key).c_str(), &v) != RTQ_OK || v == plain;
  };
  if (!kv_is(".expert_count", 0.0))
    return rtq_fail(RTQ_ERR_UNSUPPORTED, "mixture-of-experts feed-forward blocks are not trainable yet "
                                         "(dense models only)");
  if (!kv_is(".embedding_scale", 1.0) || !kv_is(".residual_scale", 1.0) || !kv_is(".logit_scale", 1.0) ||
      !kv_is(".attn_logit_softcapping", 0.0) || !kv_is(".final_logit_softcapping", 0.0) ||
      !kv_is(".attention.sliding_window", 0.0))
    return rtq_fail(RTQ_ERR_UNSUPPORTED, "%s: unsupported scaling/softcap/sliding-window settings", arch.c_str());
  // RoPE frequency scaling (rope_freq_scale, src/rie.rs:229; Rope::at_positions src/ops.rs:141-158):
  // linear scaling divides every frequency by the factor; other scaling types are refused
  {
    const char* ty = nullptr;
    uint64_t tn = 0;
    std::string type = "none";
    if (rtq_gguf_get_str(g, (arch + ".rope.scaling.type").c_str(), &ty, &tn) == RTQ_OK) type.assign(ty, tn);
    const double factor = kv_num(g, arch + ".rope.scaling.factor", 0.0);
    const double legacy = kv_num(g, arch + ".rope.scale_linear", 0.0);
    if (type == "linear" && factor > 0.0) c.rope_freq_scale = (float)(1.0 / factor);
    else if (type == "none" && legacy > 0.0) c.rope_freq_scale = (float)(1.0 / legacy);
    else if (type != "none" && !(type == "linear" && factor == 0.0))
      return rtq_fail(RTQ_ERR_UNSUPPORTED, "%s: RoPE scaling '%s' is not supported", arch.c_str(), type.c_str());
  }
  c.rope_neox = arch != "llama";  // Qwen GGUFs rotate NEOX pairs, Llama GGUFs adjacent pairs
  c.kv_f16 = 1;                   // the loader's AttnConfig { kv_f16: true } (src/rie.rs:201)
  const int64_t te = rtq_gguf_find_tensor(g, "token_embd.weight");
  if (te < 0) return rtq_fail(RTQ_ERR_INVALID, "GGUF: missing token_embd.weight");
  {
    int64_t ne[4];
    int nd = 0;
    M_TRY(rtq_gguf_tensor(g, te, nullptr, nullptr, &nd, ne, nullptr, nullptr));
    c.n_vocab = nd >= 2 ? ne[1] : 0;
  }
  if (c.n_layer <= 0 || c.n_embd <= 0 || c.n_head <= 0 || c.n_head_kv <= 0 || c.n_head % c.n_head_kv ||
      c.head_dim <= 0 || c.head_dim > 512 || c.rope_dim <= 0 || c.rope_dim > c.head_dim || c.rope_dim % 2 ||
      c.n_ff <= 0 || c.n_vocab <= 0)
    return rtq_fail(RTQ_ERR_UNSUPPORTED, "GGUF %s: unsupported or missing model hyper-parameters", arch.c_str());
  if (!kv_is(".attention.scale", 1.0) &&
      std::fabs(kv_num(g, arch + ".attention.scale", 0.0) - 1.0 / std::sqrt((double)c.head_dim)) >= 1e-6)
    return rtq_fail(RTQ_ERR_UNSUPPORTED, "%s: unsupported scaling/softcap/sliding-window settings", arch.c_str());
  // Llama-3.1-style per-frequency divisors (rope_freqs.weight, Model::rope_factors src/model.rs:477;
  // applied in Rope::at_positions src/ops.rs:151-156)
  if (const int64_t rf = rtq_gguf_find_tensor(g, "rope_freqs.weight"); rf >= 0) {
    int type = 0;
    const void* data = nullptr;
    size_t nbytes = 0;
    M_TRY(rtq_gguf_tensor(g, rf, nullptr, &type, nullptr, nullptr, &data, &nbytes));
    if (type != RTQ_TYPE_F32 || nbytes % 4 || nbytes / 4 > (size_t)c.rope_dim / 2)
      return rtq_fail(RTQ_ERR_UNSUPPORTED, "GGUF: rope_freqs.weight must be F32 with at most %lld elements",
                      (long long)(c.rope_dim / 2));
    c.n_rope_factors = (int64_t)(nbytes / 4);
    if (factors) factors->assign((const float*)data, (const float*)data + nbytes / 4);
  }
  c.qk_norm = rtq_gguf_find_tensor(g, "blk.0.attn_q_norm.weight") >= 0;
  c.tied = rtq_gguf_find_tensor(g, "output.weight") < 0;
  for (int64_t l = 0; l < c.n_layer; l++) {  // src/rie.rs:204-206
    const std::string p = "blk." + std::to_string(l) + ".";
    if (rtq_gguf_find_tensor(g, (p + "post_attention_norm.weight").c_str()) >= 0 ||
        rtq_gguf_find_tensor(g, (p + "post_ffw_norm.weight").c_str()) >= 0)
      return rtq_fail(RTQ_ERR_UNSUPPORTED, "post-norm layers are not supported");
  }
  *out = c;
  return RTQ_OK;
}
}  // namespace

extern "C" {

rtq_status rtq_model_config_from_gguf(const rtq_gguf* g, rtq_model_config* out) {
  if (!g || !out) return rtq_fail(RTQ_ERR_INVALID, "null gguf/out");
  return parse_config(g, out, nullptr);
}

rtq_status rtq_model_from_gguf(rtq_ctx* ctx, const rtq_gguf* g, rtq_model** out) {
  if (!ctx || !g || !out) return rtq_fail(RTQ_ERR_INVALID, "null ctx/gguf/out");
  *out = nullptr;
  rtq_model_config cfg{};
  std::vector<float> factors;
  M_TRY(parse_config(g, &cfg, &factors));
  rtq_model* m = new rtq_model();
  if (const char* e = getenv("RTQ_ATTN_F32")) m->attn_f32 = atoi(e) != 0;
  if (const char* e = getenv("RTQ_ATTN_ITEMS")) m->attn_items = std::max(0, atoi(e));
  if (const char* e = getenv("RTQ_LORA_BATCH")) m->lora_batch = atoi(e) != 0;
  if (const char* e = getenv("RTQ_NORM_FUSE")) m->norm_fuse = atoi(e) != 0;
  if (const char* e = getenv("RTQ_LORA_DEFER")) m->lora_defer = atoi(e) != 0;
  if (const char* e = getenv("RTQ_STEP_GRAPH")) m->graph_on = atoi(e) != 0;
  m->ctx = ctx;
  m->cfg = cfg;
  m->rope_factors = factors;
  m->attn_hd_ok = cfg.head_dim == 64 || cfg.head_dim == 128;  // the fused attention kernels' head sizes
  const rtq_model_config& c = m->cfg;
  rtq_status st = RTQ_OK;
  auto fail_out = [&](rtq_status s) {
    rtq_model_destroy(m);
    return s;
  };
  const int64_t d = c.n_embd, qd = c.n_head * c.head_dim, kd = c.n_head_kv * c.head_dim;
  if ((st = load_weight(m, g, "token_embd.weight", c.n_vocab, d, &m->embed)) != RTQ_OK) return fail_out(st);
  if (c.tied) {
    m->head = m->embed;
  } else if ((st = load_weight(m, g, "output.weight", c.n_vocab, d, &m->head)) != RTQ_OK) {
    return fail_out(st);
  }
  if ((st = upload_vec(m, g, "output_norm.weight", d, &m->out_norm, true)) != RTQ_OK) return fail_out(st);
  m->layers.resize((size_t)c.n_layer);
  const int64_t outs[NLIN] = {qd, kd, kd, d, c.n_ff, c.n_ff, d}, ins[NLIN] = {d, d, d, qd, d, d, c.n_ff};
  for (int64_t l = 0; l < c.n_layer; l++) {
    Layer& L = m->layers[(size_t)l];
    const std::string p = "blk." + std::to_string(l) + ".";
    if ((st = upload_vec(m, g, p + "attn_norm.weight", d, &L.attn_norm, true)) != RTQ_OK ||
        (st = upload_vec(m, g, p + "ffn_norm.weight", d, &L.ffn_norm, true)) != RTQ_OK ||
        (st = upload_vec(m, g, p + "attn_q_norm.weight", c.head_dim, &L.q_norm, c.qk_norm)) != RTQ_OK ||
        (st = upload_vec(m, g, p + "attn_k_norm.weight", c.head_dim, &L.k_norm, c.qk_norm)) != RTQ_OK)
      return fail_out(st);
    if ((st = load_groups(m, g, p, L, outs, ins)) != RTQ_OK) return fail_out(st);
  }
  *out = m;
  return RTQ_OK;
}

void rtq_model_destroy(rtq_model* m) {
  if (!m) return;
  (void)hipSetDevice(rtq_ctx_device_id(m->ctx));
  (void)hipStreamSynchronize(stream_of(m));
  if (m->gexec) (void)hipGraphExecDestroy(m->gexec);
  if (m->io_host) (void)hipHostFree(m->io_host);
  for (rtq_weight* w : m->weights) rtq_weight_destroy(w);
  for (void* p : m->owned) (void)hipFree(p);
  if (m->step_mem) (void)hipFree(m->step_mem);
  if (m->hpk_mem) (void)hipFree(m->hpk_mem);
  if (m->lg_mem) (void)hipFree(m->lg_mem);
  if (m->lgt_mem) (void)hipFree(m->lgt_mem);
  if (m->lgt_host) (void)hipHostFree(m->lgt_host);
  if (m->attn_mem) (void)hipFree(m->attn_mem);
  if (m->seq_mem) (void)hipFree(m->seq_mem);
  delete m;
}

rtq_status rtq_model_get_config(const rtq_model* m, rtq_model_config* out) {
  if (!m || !out) return rtq_fail(RTQ_ERR_INVALID, "null model/out");
  *out = m->cfg;
  return RTQ_OK;
}

rtq_status rtq_model_attach_lora(rtq_model* m, int64_t rank, float alpha, uint32_t target_mask, uint64_t seed,
                                 int64_t* n_params) {
  if (!m || rank <= 0 || rank > 4096) return rtq_fail(RTQ_ERR_INVALID, "bad model/rank");
  M_HIP(hipSetDevice(rtq_ctx_device_id(m->ctx)));
  M_HIP(hipStreamSynchronize(stream_of(m)));
  // the new block layout of each group's adapter (members in linear order, r columns each if
  // targeted), computed before anything changes; every adapter's dA and dB in one allocation, so
  // zero_grad is one fill
  struct Plan {
    int64_t rank = 0, col0[3] = {}, r[3] = {};
    void *A = nullptr, *B = nullptr;
  };
  std::vector<std::vector<Plan>> plan(m->layers.size());
  size_t gbytes = 0;
  for (size_t l = 0; l < m->layers.size(); l++)
    for (const Group& G : m->layers[l].groups) {
      Plan p;
      for (int j = 0; j < G.nm; j++) {
        p.col0[j] = p.rank;
        p.r[j] = (target_mask >> G.mem[j].lin & 1u) ? rank : 0;
        p.rank += p.r[j];
      }
      gbytes += ((size_t)(p.rank * G.in) * 4 + 255) / 256 * 256 + ((size_t)(G.rows * p.rank) * 4 + 255) / 256 * 256;
      plan[l].push_back(p);
    }
  // allocate everything first: a failure leaves the previous adapters as they were
  std::vector<void*> fresh;
  auto undo = [&](rtq_status st) {
    for (void* p : fresh) dev_free(m, p);
    return st;
  };
  void* gmem = nullptr;
  rtq_status st = dev_alloc(m, gbytes, &gmem);
  if (st != RTQ_OK) return undo(st);
  fresh.push_back(gmem);
  for (size_t l = 0; l < m->layers.size(); l++)
    for (size_t gi = 0; gi < m->layers[l].groups.size(); gi++) {
      Plan& p = plan[l][gi];
      const Group& G = m->layers[l].groups[gi];
      if (p.rank == 0) continue;
      if ((st = dev_alloc(m, (size_t)(p.rank * G.in) * 4, &p.A)) != RTQ_OK) return undo(st);
      fresh.push_back(p.A);
      if ((st = dev_alloc(m, (size_t)(G.rows * p.rank) * 4, &p.B)) != RTQ_OK) return undo(st);
      fresh.push_back(p.B);
    }
  if (hipMemset(gmem, 0, gbytes) != hipSuccess) return undo(rtq_fail(RTQ_ERR_HIP, "hipMemset of adapter gradients"));
  // A ~ U(+-1/sqrt(in)) drawn linear by linear in the reference's order (Lora::new, src/linear.rs:21-25), B = 0
  Rng rng(seed);
  int64_t n = 0;
  for (size_t l = 0; l < m->layers.size(); l++) {
    Layer& L = m->layers[l];
    std::vector<std::vector<float>> ahost(L.groups.size());
    for (int i = 0; i < NLIN; i++) {
      if (!(target_mask >> i & 1u)) continue;
      const Group& G = L.groups[(size_t)L.gi[i]];
      const Plan& p = plan[l][(size_t)L.gi[i]];
      std::vector<float>& a = ahost[(size_t)L.gi[i]];
      a.resize((size_t)(p.rank * G.in), 0.0f);
      const float bound = 1.0f / sqrtf((float)G.in);
      for (int64_t e = 0; e < rank * G.in; e++) a[(size_t)(p.col0[L.mi[i]] * G.in + e)] = rng.uniform_sym(bound);
      n += rank * (G.in + G.mem[L.mi[i]].rows);
    }
    for (size_t gi = 0; gi < L.groups.size(); gi++) {
      const Plan& p = plan[l][gi];
      const Group& G = L.groups[gi];
      if (p.rank == 0) continue;
      if (hipMemcpy(p.A, ahost[gi].data(), (size_t)(p.rank * G.in) * 4, hipMemcpyHostToDevice) != hipSuccess ||
          hipMemset(p.B, 0, (size_t)(G.rows * p.rank) * 4) != hipSuccess)
        return undo(rtq_fail(RTQ_ERR_HIP, "adapter upload failed"));
    }
  }
  // commit: the previous adapters' memory is released, the new layout takes their place
  dev_free(m, m->grads);
  char* gp = (char*)gmem;
  for (size_t l = 0; l < m->layers.size(); l++)
    for (size_t gi = 0; gi < m->layers[l].groups.size(); gi++) {
      Group& G = m->layers[l].groups[gi];
      const Plan& p = plan[l][gi];
      dev_free(m, G.A);
      dev_free(m, G.B);
      G.rank = p.rank;
      int members = 0;
      for (int j = 0; j < G.nm; j++) {
        G.mem[j].col0 = p.col0[j];
        G.mem[j].r = p.r[j];
        members += p.r[j] > 0;
      }
      G.alpha = alpha * (float)members;  // alpha / rank unchanged
      G.A = (float*)p.A;
      G.B = (float*)p.B;
      G.ga = G.gb = nullptr;
      if (p.rank == 0) continue;
      const size_t na = (size_t)(p.rank * G.in) * 4, nb = (size_t)(G.rows * p.rank) * 4;
      G.ga = (float*)gp;
      gp += (na + 255) / 256 * 256;
      G.gb = (float*)gp;
      gp += (nb + 255) / 256 * 256;
    }
  m->grads = gmem;
  m->gen++;
  m->grad_bytes = gbytes;
  if (n_params) *n_params = n;
  return RTQ_OK;
}

int64_t rtq_model_lora_count(const rtq_model* m) {
  int64_t n = 0;
  if (m)
    for (const Layer& L : m->layers)
      for (const Group& G : L.groups)
        for (int j = 0; j < G.nm; j++) n += G.mem[j].r > 0;
  return n;
}

namespace {
// adapter i in (block, linear) order: its group and member
bool lora_at(const rtq_model* m, int64_t i, int* layer, int* which, const Group** grp, const Member** mem) {
  if (!m || i < 0) return false;
  for (size_t l = 0; l < m->layers.size(); l++) {
    const Layer& L = m->layers[l];
    for (int k = 0; k < NLIN; k++) {
      const Group& G = L.groups[(size_t)L.gi[k]];
      const Member& mb = G.mem[L.mi[k]];
      if (mb.r > 0 && i-- == 0) {
        if (layer) *layer = (int)l;
        if (which) *which = k;
        *grp = &G;
        *mem = &mb;
        return true;
      }
    }
  }
  return false;
}
}  // namespace

rtq_status rtq_model_lora_info(const rtq_model* m, int64_t i, int* layer, int* which, int64_t* rank, int64_t* in,
                               int64_t* out, float* alpha) {
  const Group* G;
  const Member* mb;
  if (!lora_at(m, i, layer, which, &G, &mb)) return rtq_fail(RTQ_ERR_INVALID, "adapter %lld out of range", (long long)i);
  if (rank) *rank = mb->r;
  if (in) *in = G->in;
  if (out) *out = mb->rows;
  if (alpha) *alpha = G->alpha * (float)mb->r / (float)G->rank;
  return RTQ_OK;
}

rtq_status rtq_model_lora_device(rtq_model* m, int64_t i, float** a, float** b, float** ga, float** gb, int64_t* ldb) {
  const Group* G;
  const Member* mb;
  if (!lora_at(m, i, nullptr, nullptr, &G, &mb)) return rtq_fail(RTQ_ERR_INVALID, "adapter %lld out of range", (long long)i);
  const int64_t ao = mb->col0 * G->in, bo = mb->row0 * G->rank + mb->col0;
  if (a) *a = G->A + ao;
  if (b) *b = G->B + bo;
  if (ga) *ga = G->ga + ao;
  if (gb) *gb = G->gb + bo;
  if (ldb) *ldb = G->rank;
  return RTQ_OK;
}

rtq_status rtq_model_lora_get(rtq_model* m, int64_t i, float* a, float* b, float* ga, float* gb) {
  const Group* G;
  const Member* mb;
  if (!lora_at(m, i, nullptr, nullptr, &G, &mb)) return rtq_fail(RTQ_ERR_INVALID, "adapter %lld out of range", (long long)i);
  M_HIP(hipSetDevice(rtq_ctx_device_id(m->ctx)));
  M_HIP(hipStreamSynchronize(stream_of(m)));
  const int64_t ao = mb->col0 * G->in, bo = mb->row0 * G->rank + mb->col0;
  const size_t na = (size_t)(mb->r * G->in) * 4, w = (size_t)mb->r * 4, ld = (size_t)G->rank * 4;
  if (a) M_HIP(hipMemcpy(a, G->A + ao, na, hipMemcpyDeviceToHost));
  if (ga) M_HIP(hipMemcpy(ga, G->ga + ao, na, hipMemcpyDeviceToHost));
  if (b) M_HIP(hipMemcpy2D(b, w, G->B + bo, ld, w, (size_t)mb->rows, hipMemcpyDeviceToHost));
  if (gb) M_HIP(hipMemcpy2D(gb, w, G->gb + bo, ld, w, (size_t)mb->rows, hipMemcpyDeviceToHost));
  return RTQ_OK;
}

rtq_status rtq_model_lora_set(rtq_model* m, int64_t i, const float* a, const float* b) {
  const Group* G;
  const Member* mb;
  if (!lora_at(m, i, nullptr, nullptr, &G, &mb)) return rtq_fail(RTQ_ERR_INVALID, "adapter %lld out of range", (long long)i);
  M_HIP(hipSetDevice(rtq_ctx_device_id(m->ctx)));
  M_HIP(hipStreamSynchronize(stream_of(m)));
  const int64_t ao = mb->col0 * G->in, bo = mb->row0 * G->rank + mb->col0;
  const size_t w = (size_t)mb->r * 4, ld = (size_t)G->rank * 4;
  if (a) M_HIP(hipMemcpy(G->A + ao, a, (size_t)(mb->r * G->in) * 4, hipMemcpyHostToDevice));
  if (b) M_HIP(hipMemcpy2D(G->B + bo, ld, b, w, w, (size_t)mb->rows, hipMemcpyHostToDevice));
  return RTQ_OK;
}

rtq_status rtq_model_zero_grad(rtq_model* m) {
  if (!m) return rtq_fail(RTQ_ERR_INVALID, "null model");
  M_HIP(hipSetDevice(rtq_ctx_device_id(m->ctx)));
  if (m->grads) M_HIP(hipMemsetAsync(m->grads, 0, m->grad_bytes, stream_of(m)));  // every adapter's dA, dB
  M_HIP(hipStreamSynchronize(stream_of(m)));
  return RTQ_OK;
}

}  // extern "C"

namespace {
// the kernels of a step (forward_backward_layout, src/model.rs:644-687): embed, blocks (activations
// kept, or only the block inputs when recomputing), head, blocks in reverse (recomputing each
// block's forward first).  Inputs are on the device; nothing here allocates or synchronises once an
// identical step has run before (its buffers, job tables and workspace are in place), so it can be
// captured into a graph.
rtq_status step_kernels(rtq_model* m, int64_t t, int64_t n, bool weights) {
  const rtq_model_config& c = m->cfg;
  hipStream_t st = stream_of(m);
  const int64_t d = c.n_embd;
  M_TRY(rtq_frozen_gather_d(m->ctx, m->embed, m->tok_d, t, m->X, st));  // embed_tokens
  bool pending = false;  // block l's output sum left to block l + 1's first norm
  for (int64_t l = 0; l < c.n_layer; l++) {
    float *x = m->X + l * t * d, *y = m->X + (l + 1) * t * d;
    // the residual sum of a block's output is formed by the next block's first norm, except where
    // the output itself is read next (the last block: the LM head; a captured block)
    const bool out = l == c.n_layer - 1 || l == m->dbg_layer;
    M_TRY(block_forward(m, (int)l, t, x, y, pending, out));
    pending = !out;
    if (l == m->dbg_layer) M_TRY(dbg_forward(m, (int)l, t, x, y));
  }
  if (n == 0) return RTQ_OK;
  M_TRY(rtq_lm_head_d(m->ctx, m->head, m->out_norm, c.rms_eps, c.norm_offset, m->X + c.n_layer * t * d, t, m->pos_d,
                      m->tgt_d, weights ? m->wts_d : nullptr, n, m->logp_d, m->hit_d, weights ? m->dY : nullptr, st));
  if (!weights) return RTQ_OK;
  m->lg_all.clear();
  for (int64_t l = c.n_layer - 1; l >= 0; l--) {
    const float* x = m->X + l * t * d;
    if (m->ckpt) M_TRY(block_forward(m, (int)l, t, const_cast<float*>(x), m->f, false, false));  // recompute
    // deferring: each block's input gradient stays in its own buffer (the block below reads it
    // as its dy, the deferred dB of its down projection at the end)
    float* gy = m->defer_lg && l < c.n_layer - 1 ? m->cache[(size_t)l + 1].gx : m->dY;
    float* gx = m->defer_lg ? m->cache[(size_t)l].gx : m->dX;
    M_TRY(block_backward(m, (int)l, t, x, gy, gx));
    if (l == m->dbg_layer) M_TRY(dbg_backward(m, (int)l, t, gy, gx));
    if (!m->defer_lg) std::swap(m->dY, m->dX);
  }
  if (m->defer_lg) M_TRY(lora_grads_all(m));
  return RTQ_OK;
}

// captures step_kernels into the model's graph (replacing the one it held) and launches it.  A
// step that cannot be captured (the runtime refuses an operation in it) runs eagerly, and the model
// stays eager from then on.
rtq_status capture_step(rtq_model* m, int64_t t, int64_t n, bool weights, const std::vector<uint64_t>& key) {
  hipStream_t st = stream_of(m);
  if (m->gexec) {
    M_HIP(hipGraphExecDestroy(m->gexec));
    m->gexec = nullptr;
    m->gkey.clear();
  }
  const char* why = nullptr;
  if (hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal) != hipSuccess) {
    why = "hipStreamBeginCapture";
  } else {
    const rtq_status s = step_kernels(m, t, n, weights);
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(st, &g);
    hipGraphExec_t x = nullptr;
    if (s != RTQ_OK || e != hipSuccess || !g) why = s != RTQ_OK ? rtq_last_error() : "hipStreamEndCapture";
    else if (hipGraphInstantiate(&x, g, nullptr, nullptr, 0) != hipSuccess) why = "hipGraphInstantiate";
    if (g) (void)hipGraphDestroy(g);
    if (!why) {
      m->gexec = x;
      m->gkey = key;
      M_HIP(hipGraphLaunch(x, st));
      return RTQ_OK;
    }
  }
  (void)hipGetLastError();
  fprintf(stderr, "rtq: the step could not be captured as a graph (%s); steps run eagerly\n", why);
  m->graph_on = false;
  return step_kernels(m, t, n, weights);
}

// one step (forward_backward_layout, src/model.rs:644-687): checks, buffers and tables, the
// inputs' upload, the kernels (eager, captured or replayed), the outputs' download
rtq_status step(rtq_model* m, const int32_t* tokens, int64_t t, const int32_t* positions, const int32_t* segments,
                const int32_t* pos, const int32_t* tok, const float* weights, int64_t n, float* logp, int64_t* hits) {
  if (!m || !tokens || t <= 0 || n < 0 || (n > 0 && (!pos || !tok || !logp)))
    return rtq_fail(RTQ_ERR_INVALID, "null model/tokens/targets or empty sequence");
  const rtq_model_config& c = m->cfg;
  if (t > 65535) return rtq_fail(RTQ_ERR_INVALID, "sequence of %lld tokens too long", (long long)t);
  for (int64_t i = 0; i < t; i++)
    if (tokens[i] < 0 || tokens[i] >= c.n_vocab)
      return rtq_fail(RTQ_ERR_INVALID, "token %d out of vocab", tokens[i]);  // src/model.rs:450
  for (int64_t i = 0; i < n; i++)
    if (pos[i] < 0 || pos[i] >= t || tok[i] < 0 || tok[i] >= c.n_vocab)
      return rtq_fail(RTQ_ERR_INVALID, "target %lld out of range", (long long)i);  // src/model.rs:575
  if (positions)
    for (int64_t i = 0; i < t; i++)
      if (positions[i] < 0) return rtq_fail(RTQ_ERR_INVALID, "position %lld is negative", (long long)i);
  if (segments)
    for (int64_t i = 0; i < t; i++)
      if (segments[i] < 0) return rtq_fail(RTQ_ERR_INVALID, "segment %lld is negative", (long long)i);
  M_HIP(hipSetDevice(rtq_ctx_device_id(m->ctx)));
  m->attn_fused = m->attn_hd_ok && m->attn_mode != 0;
  M_TRY(choose_ckpt(m, t, n));
  M_TRY(choose_defer(m, t));
  M_TRY(ensure_step(m, t, n));
  M_TRY(ensure_hpk(m, t));
  M_TRY(ensure_lgrad(m, t));
  M_TRY(ensure_rope(m, t, positions));
  M_TRY(upload_layout(m, segments, t));
  if (m->attn_fused) M_TRY(ensure_attn_plan(m, t, segments));
  M_TRY(ensure_seq_plan(m, t, segments));
  hipStream_t st = stream_of(m);
  // host inputs and outputs pass through pinned staging, so the copies are asynchronous; the
  // staging is free again once the step's synchronisation below returns
  const size_t io_need = (size_t)(t + 5 * n) * 4;
  if (io_need > m->io_cap) {
    if (m->io_host) M_HIP(hipHostFree(m->io_host));
    m->io_host = nullptr;
    m->io_cap = 0;
    const size_t cap = std::max<size_t>(io_need, 1 << 16);
    M_HIP(hipHostMalloc(&m->io_host, cap));
    m->io_cap = cap;
  }
  int32_t* io = (int32_t*)m->io_host;  // tokens [t] | pos [n] | tok [n] | weights [n] | logp [n] | hits [n]
  std::memcpy(io, tokens, (size_t)t * 4);
  M_HIP(hipMemcpyAsync(m->tok_d, io, (size_t)t * 4, hipMemcpyHostToDevice, st));
  if (n > 0) {
    std::memcpy(io + t, pos, (size_t)n * 4);
    std::memcpy(io + t + n, tok, (size_t)n * 4);
    M_HIP(hipMemcpyAsync(m->pos_d, io + t, (size_t)n * 4, hipMemcpyHostToDevice, st));
    M_HIP(hipMemcpyAsync(m->tgt_d, io + t + n, (size_t)n * 4, hipMemcpyHostToDevice, st));
    if (weights) {
      std::memcpy(io + t + 2 * n, weights, (size_t)n * 4);
      M_HIP(hipMemcpyAsync(m->wts_d, io + t + 2 * n, (size_t)n * 4, hipMemcpyHostToDevice, st));
    }
  }
  // the launch key: everything the step's launches depend on besides gen (bumped by the rest)
  const bool graphable = m->graph_on && m->dbg_layer < 0 && !rtq_ctx_timing_on(m->ctx);
  std::vector<uint64_t> key;
  if (graphable)
    key = {(uint64_t)t, (uint64_t)n, weights ? 1u : 0u, m->packed ? 1u : 0u, (uint64_t)m->nlb,
           m->ckpt ? 1u : 0u, m->defer_lg ? 1u : 0u, m->attn_fused ? 1u : 0u, (uint64_t)m->n_fwd,
           (uint64_t)m->n_kv, (uint64_t)m->n_mfwd, (uint64_t)m->n_mkv, m->packed && m->seq_on ? 1u : 0u,
           (uint64_t)m->tv, (uint64_t)m->n_sit, (uint64_t)m->n_smg, m->gen, rtq_ctx_ws_gen(m->ctx)};
  if (graphable && m->gexec && key == m->gkey) {
    M_HIP(hipGraphLaunch(m->gexec, st));
    m->graph_replays++;
  } else if (graphable && key == m->prev_key) {
    M_TRY(capture_step(m, t, n, weights != nullptr, key));
  } else {
    M_TRY(step_kernels(m, t, n, weights != nullptr));
  }
  m->prev_key = key;
  if (n > 0) {
    float* lp = (float*)(io + t + 3 * n);
    int32_t* hv = io + t + 4 * n;
    M_HIP(hipMemcpyAsync(lp, m->logp_d, (size_t)n * 4, hipMemcpyDeviceToHost, st));
    M_HIP(hipMemcpyAsync(hv, m->hit_d, (size_t)n * 4, hipMemcpyDeviceToHost, st));
    M_HIP(hipStreamSynchronize(st));
    std::memcpy(logp, lp, (size_t)n * 4);
    if (hits) {
      int64_t s = 0;
      for (int64_t i = 0; i < n; i++) s += hv[i];
      *hits = s;
    }
  } else {
    M_HIP(hipStreamSynchronize(st));
    if (hits) *hits = 0;
  }
  return RTQ_OK;
}
}  // namespace

extern "C" {

rtq_status rtq_model_forward_backward(rtq_model* m, const int32_t* tokens, int64_t t, const int32_t* pos,
                                      const int32_t* tok, const float* weights, int64_t n, float* logp,
                                      int64_t* hits) {
  return step(m, tokens, t, nullptr, nullptr, pos, tok, weights, n, logp, hits);
}

rtq_status rtq_model_forward_backward_packed(rtq_model* m, const int32_t* tokens, int64_t t,
                                             const int32_t* positions, const int32_t* segments, const int32_t* pos,
                                             const int32_t* tok, const float* weights, int64_t n, float* logp,
                                             int64_t* hits) {
  if (!positions || !segments) return rtq_fail(RTQ_ERR_INVALID, "packed step needs positions and segments");
  return step(m, tokens, t, positions, segments, pos, tok, weights, n, logp, hits);
}

rtq_status rtq_model_set_checkpointing(rtq_model* m, int mode) {
  if (!m || mode < -1 || mode > 1) return rtq_fail(RTQ_ERR_INVALID, "bad model/checkpointing mode %d", mode);
  m->ckpt_mode = mode;
  m->gen++;
  return RTQ_OK;
}

int rtq_model_checkpointing(const rtq_model* m) { return m ? (m->ckpt ? 1 : 0) : -1; }

rtq_status rtq_model_set_attention(rtq_model* m, int mode) {
  if (!m || mode < -1 || mode > 1) return rtq_fail(RTQ_ERR_INVALID, "bad model/attention mode %d", mode);
  m->attn_mode = mode;
  m->gen++;
  return RTQ_OK;
}

int rtq_model_attention_fused(const rtq_model* m) { return m ? (m->attn_fused ? 1 : 0) : -1; }

int64_t rtq_model_graph_replays(const rtq_model* m) { return m ? m->graph_replays : -1; }

rtq_status rtq_model_debug_capture(rtq_model* m, int64_t layer) {
  if (!m || layer < -1 || layer >= m->cfg.n_layer) return rtq_fail(RTQ_ERR_INVALID, "bad model/layer");
  m->dbg_layer = layer;
  m->gen++;
  return RTQ_OK;
}

rtq_status rtq_model_debug_tensor(rtq_model* m, const char* name, float* out, int64_t nfloats) {
  if (!m || !name) return rtq_fail(RTQ_ERR_INVALID, "null model/name");
  for (auto& e : m->dbg)
    if (e.first == name) {
      if (!out) return e.second.second > nfloats ? rtq_fail(RTQ_ERR_INVALID, "%s has %lld floats", name,
                                                            (long long)e.second.second)
                                                 : RTQ_OK;
      if (nfloats != e.second.second)
        return rtq_fail(RTQ_ERR_INVALID, "%s has %lld floats, not %lld", name, (long long)e.second.second,
                        (long long)nfloats);
      M_HIP(hipSetDevice(rtq_ctx_device_id(m->ctx)));
      M_HIP(hipStreamSynchronize(stream_of(m)));
      M_HIP(hipMemcpy(out, e.second.first, (size_t)nfloats * 4, hipMemcpyDeviceToHost));
      return RTQ_OK;
    }
  return rtq_fail(RTQ_ERR_INVALID, "no captured tensor %s", name);
}

}  // extern "C"
