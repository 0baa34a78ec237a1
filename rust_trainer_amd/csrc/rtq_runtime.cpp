// rtq_runtime.cpp — host runtime of librtq.so: the C ABI declared in include/rtq.h.
//
// Owns the HIP context pieces (device, stream, the gfx950 code object loaded with
// hipModuleLoadData from bytes embedded at build time), the device copies of the frozen weights
// in their fragment layout, and a grow-only device workspace for per-call intermediates.
// Every launch goes through hipModuleLaunchKernel with one argument block (rtq_kargs.h).
//
// There is no CPU fallback: every entry point fails with a status code when the device or the
// code object is unavailable.
#include "rtq.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "rtq_internal.h"
#include "rtq_kargs.h"

#ifndef RTQ_HSACO_PATH
#error "RTQ_HSACO_PATH must name the gfx950 code object to embed"
#endif

// The code object is embedded into the shared library so that no file lookup happens at run time.
__asm__(
    ".section .rodata.rtq_hsaco,\"a\",@progbits\n"
    ".balign 4096\n"
    ".local rtq_hsaco_begin\n"
    "rtq_hsaco_begin:\n"
    ".incbin \"" RTQ_HSACO_PATH
    "\"\n"
    ".local rtq_hsaco_end\n"
    "rtq_hsaco_end:\n"
    ".byte 0\n"
    ".previous\n");
extern "C" const char rtq_hsaco_begin[];
extern "C" const char rtq_hsaco_end[];

namespace {

thread_local std::string g_err;

rtq_status fail(rtq_status st, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return st;
}

#define HIP_TRY(expr)                                                                              \
  do {                                                                                             \
    hipError_t e_ = (expr);                                                                        \
    if (e_ != hipSuccess) return fail(RTQ_ERR_HIP, "%s: %s (%s:%d)", #expr, hipGetErrorString(e_), \
                                      __FILE__, __LINE__);                                         \
  } while (0)

#define RTQ_TRY(expr)              \
  do {                             \
    rtq_status s_ = (expr);        \
    if (s_ != RTQ_OK) return s_;   \
  } while (0)

inline int64_t roundup(int64_t a, int64_t b) { return (a + b - 1) / b * b; }
inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

uint16_t f32_to_f16_bits(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
  if (ax < 0x38800000u) {
    float af;
    memcpy(&af, &ax, 4);
    return (uint16_t)(sign | (uint32_t)__builtin_nearbyintf(af * 16777216.0f));
  }
  uint32_t e = (ax >> 23) - 112, mant = ax & 0x7fffffu, h = (e << 10) | (mant >> 13), rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return (uint16_t)(sign | h);
}

float f16_bits_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  uint32_t bits;
  if (e == 0) {
    float v = (float)m * (1.0f / 16777216.0f);
    memcpy(&bits, &v, 4);
    bits |= sign;
  } else if (e == 31) {
    bits = sign | 0x7f800000u | (m << 13);
  } else {
    bits = sign | ((e + 112) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

// format index of the per-format kernel tables: Q4_0, Q8_0, Q4_K, Q6_K
enum { F_Q4_0, F_Q8_0, F_Q4_K, F_Q6_K, F_COUNT };

enum Kid {
  K_FILL,
  K_ACT_PREP,    // Q8_0 activations (Q4_0, Q8_0 weights)
  K_ACT_PREP_K,  // Q8_K activations (Q4_K, Q6_K weights)
  K_FWD_W,       // + format: wide forward GEMM
  K_FWD_S = K_FWD_W + F_COUNT,            // skinny (t <= 16)
  K_FWD_W_ISUMS = K_FWD_S + F_COUNT,      // debug variants writing the integer sums
  K_FWD_S_ISUMS = K_FWD_W_ISUMS + F_COUNT,
  K_GEMV = K_FWD_S_ISUMS + F_COUNT,       // + format: t <= 16, large N
  K_GEMVQ1 = K_GEMV + F_COUNT,            // + format: t == 1, one launch (its own activation codes)
  K_GEMVQ4 = K_GEMVQ1 + F_COUNT,          // + format: t <= 4, one launch
  K_FWD_Q4_0_W8 = K_GEMVQ4 + F_COUNT,     // wide forward with eight waves splitting K
  K_FWD_Q8_0_W8,
  K_FWD_Q4_0_W8R2,  // the same with 32-row tiles
  K_FWD_Q8_0_W8R2,
  K_FWD_Q4_0_W8R1,  // the same with 16-row tiles
  K_FWD_Q8_0_W8R1,
  K_MM_Q4_0,     // large-grid forward (128 x 128 tiles, LDS ring)
  K_MM_Q8_0,
  K_MM64_Q4_0,   // the same with 128 x 64 tiles
  K_MM64_Q8_0,
  K_MM32_Q4_0,   // the same with 128 x 32 tiles
  K_MM32_Q8_0,
  K_MMI8_64_Q4_0,  // the 128 x 64 tiles with the block sums on int8 MFMA
  K_MMI8_64_Q8_0,
  K_MMK64_Q4_K,    // the LDS-ring kernel for the K-quants: 128 x 64 and 128 x 32 tiles
  K_MMK64_Q6_K,
  K_MMK32_Q4_K,
  K_MMK32_Q6_K,
  K_BWD_PREP,
  K_DX,          // + format
  K_DX16 = K_DX + F_COUNT,  // + format: t <= 16
  K_DXV1 = K_DX16 + F_COUNT,  // + format: t == 1, f32 FMAs
  K_DXW = K_DXV1 + F_COUNT,  // + format: large t, 256-token tiles
  K_DX32 = K_DXW + F_COUNT,  // + format: 32-token tiles on four-wave workgroups
  K_BWD_FINISH = K_DX32 + F_COUNT,
  K_BWD_FINISH16,  // 16 waves per workgroup: long token reductions of dA / dB
  K_BWD_FINISH_DX,  // dx workgroups alone (no dA / dB tiles in the grid)
  K_BWD_FINISH_ROWS,  // row-major partials of many splits: a workgroup per (token, 64 columns)
  K_LORA_GRADS,    // dA / dB of several linears in one launch (4 / 16 waves per workgroup)
  K_LORA_GRADS16,
  K_LORA_GRADS_T,    // the same from a device job table
  K_LORA_GRADS_T16,
  K_DENSE_ROWS,    // trainer-native weights: rows / dequantisation, bias
  K_DENSE_BIAS,
  K_HEAD_NORM,   // LM head + cross-entropy (Model::head)
  K_HEAD_MAX,
  K_HEAD_SUM,
  K_HEAD_GRAD,
  K_HEAD_NORM_BWD,
  K_ACT_PREP8,   // Q8_0 activations of the block norms on 8-token tiles
  K_ACT_PREP4,   // the same on 4-token tiles
  K_ROWS,        // + format
  K_MODEL = K_ROWS + F_COUNT,  // + RtqModelKernel: the decoder block (rtq_model.cpp)
  K_COUNT = K_MODEL + KM_COUNT
};
constexpr const char* kKernelNames[] = {
    "rtq_fill_zero",        "rtq_act_prep_q8_0",    "rtq_act_prep_q8_k",
    "rtq_fwd_q4_0_w",       "rtq_fwd_q8_0_w",       "rtq_fwd_q4_k_w",       "rtq_fwd_q6_k_w",
    "rtq_fwd_q4_0_s",       "rtq_fwd_q8_0_s",       "rtq_fwd_q4_k_s",       "rtq_fwd_q6_k_s",
    "rtq_fwd_q4_0_w_isums", "rtq_fwd_q8_0_w_isums", "rtq_fwd_q4_k_w_isums", "rtq_fwd_q6_k_w_isums",
    "rtq_fwd_q4_0_s_isums", "rtq_fwd_q8_0_s_isums", "rtq_fwd_q4_k_s_isums", "rtq_fwd_q6_k_s_isums",
    "rtq_gemv_q4_0",        "rtq_gemv_q8_0",        "rtq_gemv_q4_k",        "rtq_gemv_q6_k",
    "rtq_gemvq1_q4_0",      "rtq_gemvq1_q8_0",      "rtq_gemvq1_q4_k",      "rtq_gemvq1_q6_k",
    "rtq_gemvq4_q4_0",      "rtq_gemvq4_q8_0",      "rtq_gemvq4_q4_k",      "rtq_gemvq4_q6_k",
    "rtq_fwd_q4_0_w8",      "rtq_fwd_q8_0_w8",      "rtq_fwd_q4_0_w8r2",    "rtq_fwd_q8_0_w8r2",
    "rtq_fwd_q4_0_w8r1",    "rtq_fwd_q8_0_w8r1",
    "rtq_mm_q4_0",          "rtq_mm_q8_0",
    "rtq_mm64_q4_0",        "rtq_mm64_q8_0",        "rtq_mm32_q4_0",        "rtq_mm32_q8_0",
    "rtq_mmi8_64_q4_0",     "rtq_mmi8_64_q8_0",
    "rtq_mmk64_q4_k",       "rtq_mmk64_q6_k",       "rtq_mmk32_q4_k",       "rtq_mmk32_q6_k",
    "rtq_bwd_prep",
    "rtq_dx_q4_0",          "rtq_dx_q8_0",          "rtq_dx_q4_k",          "rtq_dx_q6_k",
    "rtq_dx16_q4_0",        "rtq_dx16_q8_0",        "rtq_dx16_q4_k",        "rtq_dx16_q6_k",
    "rtq_dxv1_q4_0",        "rtq_dxv1_q8_0",        "rtq_dxv1_q4_k",        "rtq_dxv1_q6_k",
    "rtq_dxw_q4_0",         "rtq_dxw_q8_0",         "rtq_dxw_q4_k",         "rtq_dxw_q6_k",
    "rtq_dx32_q4_0",        "rtq_dx32_q8_0",        "rtq_dx32_q4_k",        "rtq_dx32_q6_k",
    "rtq_bwd_finish",       "rtq_bwd_finish16",     "rtq_bwd_finish_dx",    "rtq_bwd_finish_rows",  "rtq_lora_grads",       "rtq_lora_grads16",     "rtq_lora_grads_t",     "rtq_lora_grads_t16",
    "rtq_dense_rows",       "rtq_dense_bias",
    "rtq_head_norm",        "rtq_head_max",         "rtq_head_sum",         "rtq_head_grad",
    "rtq_head_norm_bwd",    "rtq_act_prep8_q8_0",   "rtq_act_prep4_q8_0",
    "rtq_rows_q4_0",        "rtq_rows_q8_0",        "rtq_rows_q4_k",        "rtq_rows_q6_k",
    "rtq_m_rmsnorm",        "rtq_m_rmsnorm_bwd",    "rtq_m_qk_prep",        "rtq_m_qk_bwd",
    "rtq_m_gemm",           "rtq_m_softmax",        "rtq_m_softmax_bwd",    "rtq_m_group_sum",
    "rtq_m_swiglu",         "rtq_m_swiglu_bwd",     "rtq_m_add",            "rtq_m_gemm32",
    "rtq_m_lora_mask",      "rtq_m_gemm32g",        "rtq_m_gemm_q8",        "rtq_m_gemm32_q8",
    "rtq_m_attn_merge_fwd", "rtq_m_attn_merge_bwd",
    "rtq_m_attn_bwd_prep64", "rtq_m_gemm_bf",       "rtq_m_gemm32_bf",
    "rtq_m_gemm32g_bf",     "rtq_m_gemm_hf",        "rtq_m_gemm32_hf",      "rtq_m_fa_fwd64",
    "rtq_m_fa_fwd128",      "rtq_m_fa_bwd64",       "rtq_m_fa_bwd128",      "rtq_m_attn_bwd_prep128",
    "rtq_m_seq_gather",     "rtq_m_seq_scatter"};
static_assert(sizeof(kKernelNames) / sizeof(kKernelNames[0]) == K_COUNT, "one name per kernel id, in id order");

struct TimedLaunch {
  int kid;
  hipEvent_t a, b;
  double flops, bytes;  // algorithmic work of the launch (0 for kernels without a work model)
};

}  // namespace

struct rtq_ctx {
  int device = 0;
  int cu_count = 256;
  hipModule_t mod = nullptr;
  hipFunction_t fn[K_COUNT] = {};
  hipStream_t stream = nullptr;
  std::mutex mu;
  void* ws = nullptr;
  size_t ws_bytes = 0;
  uint64_t ws_gen = 0;  // bumped whenever ws moves (graphs that captured its address are stale)
  bool timing = false;
  int timing_only = -1;  // -1: every kernel
  std::vector<TimedLaunch> pending;
  std::vector<hipEvent_t> free_events;
  int dx_splits = 0;  // 0: automatic; RTQ_DX_SPLITS overrides (tuning)
  int gtok = 0;       // g-partial tokens per workgroup: 0 automatic, else 16 / 32 / 64 (RTQ_GTOK)
  int dx_wpc = 1;     // 64-token dx tiles: row splits for about this many workgroups per CU (RTQ_DX_WPC)
  int dx_wide = -1;   // 256-token dx tiles: -1 automatic, 0 never, 1 for every t > 16 (RTQ_DX_WIDE)
  int dx_32 = 0;      // 32-token dx tiles (RTQ_DX_32): 0 never, 1 with the 64-token plan's splits, 2 with
                      // half of them
  int fwd_waves = 8;  // waves splitting K in the wide Q4_0 / Q8_0 forward (RTQ_FWD_WAVES: 4 or 8)
  int fwd_rg = -1;    // row groups of 16 per eight-wave forward tile: -1 automatic, 1, 2 or 3 (RTQ_FWD_RG)
  int act_tt = 8;     // token tile of the block norms' Q8_0 activation kernel: 16, 8 or 4 (RTQ_ACT_TT;
                      // configs[2] step, activation kernels: 1.11 / 0.97-1.00 / 1.08 ms)
  int g64_min = -1;   // fewest 64-token g-partial workgroups (else 16-token ones): -1 = CUs / 2 (RTQ_G64_MIN)
  int fwd_mm = -1;    // large-grid forward: -1 automatic, 0 never, 1 / 2 / 3 the 128- / 64- / 32-token tiles
                      // whenever the format allows (RTQ_FWD_MM)
  int fwd_mmk = -1;   // K-quant ring forward (rtq_mmk*_*; RTQ_FWD_MMK): -1 automatic, 0 never, 1 / 2 the 64- /
                      // 32-token tiles whenever the shape allows
  int dxv = 1;        // t == 1 dx on f32 FMAs (rtq_dxv1_*; RTQ_DXV=0: rtq_dx16_*)
  int dxv_wpc = 3;    // rtq_dxv1_* row splits for about this many workgroups per CU (RTQ_DXV_WPC)
  int gemvq = 1;      // one-launch GEMV for t <= 4 (rtq_gemvq*_*; RTQ_GEMVQ=0: activation kernel + GEMM)
  int gemvq_wpc = 0;  // its waves per CU (RTQ_GEMVQ_WPC; 0: automatic)
  int fwd_i8 = -1;    // int8-MFMA forwards (rtq_mmi8_*; RTQ_FWD_I8): -1 automatic (Q8_0 weights), 0 never,
                      // 1 every Q4_0 / Q8_0 weight, wherever the 128- or 64-token tiles are chosen
  int64_t t_launches[K_COUNT] = {};
  double t_ms[K_COUNT] = {};
  double t_flops[K_COUNT] = {}, t_bytes[K_COUNT] = {};
  // algorithmic work of the next launch (set_work), attached to its timing record
  double next_flops = 0.0, next_bytes = 0.0;
};

struct rtq_weight {
  rtq_ctx* ctx = nullptr;
  int type = 0;
  int64_t rows = 0, cols = 0;  // N, K
  int64_t Np = 0, Kp = 0;
  size_t gguf_bytes = 0;
  void* dmem = nullptr;
  void* wq = nullptr;
  uint16_t* wd = nullptr;
  uint16_t* wdr = nullptr;  // row-major scales for the GEMV (the K-quants' wd itself)
  uint32_t* wsb = nullptr;  // K-quant super-block scales, else null
  const float* wsc = nullptr;  // TQ8_0: f32 block scales (wq: the i8 codes; F32: wq is the weight)
  // the dx kernels' f16 range: dequantised values times dx_wsc = 2^-sigma stay below 2^15 (sigma 0
  // unless a scale is huge); their partials are multiplied by dx_wunsc = 2^sigma
  float dx_wsc = 1.0f, dx_wunsc = 1.0f;
};

namespace {

// ------------------------------------------------------------------ launching
hipEvent_t get_event(rtq_ctx* c) {
  if (!c->free_events.empty()) {
    hipEvent_t e = c->free_events.back();
    c->free_events.pop_back();
    return e;
  }
  // timing-only events without the system-scope fence (no cache writeback and invalidation in the
  // recorded interval); an interval still reads about 3.5 us longer than the kernel-trace duration
  hipEvent_t e = nullptr;
  if (hipEventCreateWithFlags(&e, hipEventDisableSystemFence) != hipSuccess) return nullptr;
  return e;
}

rtq_status launch_raw(rtq_ctx* c, int kid, dim3 grid, dim3 block, hipStream_t s, void* argp, unsigned shmem) {
  if (grid.x == 0 || grid.y == 0 || grid.z == 0) return RTQ_OK;
  if (grid.y > 65535 || grid.z > 65535)
    return fail(RTQ_ERR_INVALID, "%s: grid (%u,%u,%u) out of range", kKernelNames[kid], grid.x, grid.y, grid.z);
  void* params[] = {argp};
  hipEvent_t ea = nullptr, eb = nullptr;
  const bool timed = c->timing && (c->timing_only < 0 || c->timing_only == kid);
  if (timed) {
    ea = get_event(c);
    eb = get_event(c);
    if (ea && eb) HIP_TRY(hipEventRecord(ea, s));
  }
  hipError_t e = hipModuleLaunchKernel(c->fn[kid], grid.x, grid.y, grid.z, block.x, block.y, block.z, shmem, s,
                                       params, nullptr);
  if (e != hipSuccess) return fail(RTQ_ERR_HIP, "launch %s: %s", kKernelNames[kid], hipGetErrorString(e));
  if (timed && ea && eb) {
    HIP_TRY(hipEventRecord(eb, s));
    c->pending.push_back({kid, ea, eb, c->next_flops, c->next_bytes});
  }
  c->next_flops = c->next_bytes = 0.0;
  return RTQ_OK;
}

template <class Args>
rtq_status launch(rtq_ctx* c, int kid, dim3 grid, dim3 block, hipStream_t s, const Args& args, unsigned shmem = 0) {
  Args copy = args;
  return launch_raw(c, kid, grid, block, s, &copy, shmem);
}

// the algorithmic work of a frozen-linear call (each operand touched once), recorded with the next
// launch's timing: forward = packed W + x + y + A, B (f32) and 2 T N K + the LoRA products; dx =
// packed W + dy + dx and 2 T N K
void set_work(rtq_ctx* c, const rtq_weight* w, int64_t t, int64_t r, bool backward);

// ------------------------------------------------------------------ workspace
struct Arena {
  char* base;
  size_t cap, off;
  template <class T>
  T* take(size_t count) {
    off = roundup((int64_t)off, 256);
    T* p = reinterpret_cast<T*>(base + off);
    off += count * sizeof(T);
    return p;
  }
};

// grows the context workspace to at least `bytes` (synchronises the device before freeing)
rtq_status ensure_ws(rtq_ctx* c, size_t bytes) {
  if (bytes <= c->ws_bytes) return RTQ_OK;
  size_t want = std::max<size_t>(bytes + bytes / 4, 1 << 20);
  if (c->ws) {
    HIP_TRY(hipDeviceSynchronize());
    HIP_TRY(hipFree(c->ws));
    c->ws = nullptr;
    c->ws_bytes = 0;
  }
  HIP_TRY(hipMalloc(&c->ws, want));
  c->ws_bytes = want;
  c->ws_gen++;
  return RTQ_OK;
}

bool is_q32(int type) { return type == RTQ_TYPE_Q4_0 || type == RTQ_TYPE_Q8_0; }
bool is_kquant(int type) { return type == RTQ_TYPE_Q4_K || type == RTQ_TYPE_Q6_K; }
// trainer-native FrozenWeight storage: f32 products on the f32 MFMA GEMM
bool is_dense(int type) { return type == RTQ_TYPE_F32 || type == RTQ_TYPE_TQ8_0; }
bool supported(int type) { return is_q32(type) || is_kquant(type) || is_dense(type); }
int fmt_index(int type) {
  switch (type) {
    case RTQ_TYPE_Q4_0: return F_Q4_0;
    case RTQ_TYPE_Q8_0: return F_Q8_0;
    case RTQ_TYPE_Q4_K: return F_Q4_K;
    default: return F_Q6_K;
  }
}
// device codes are bytes (Q8_0 layout) for Q8_0 and Q6_K, nibbles (Q4_0 layout) otherwise
bool byte_codes(int type) { return type == RTQ_TYPE_Q8_0 || type == RTQ_TYPE_Q6_K; }

int64_t block_elems(int type) { return type == RTQ_TYPE_F32 ? 1 : (is_q32(type) || type == RTQ_TYPE_TQ8_0 ? 32 : 256); }
int64_t block_bytes(int type) {
  switch (type) {
    case RTQ_TYPE_F32: return 4;
    case RTQ_TYPE_TQ8_0: return 36;  // f32 scale + 32 codes (stored as two arrays)
    case RTQ_TYPE_Q4_0: return 18;
    case RTQ_TYPE_Q8_0: return 34;
    case RTQ_TYPE_Q4_K: return 144;
    case RTQ_TYPE_Q6_K: return 210;
  }
  return 0;
}

// ------------------------------------------------------------------ per-call sizes
// Forward: tokens padded to 16 (skinny kernel, t <= 16) or 64 (wide kernel).
// The activation kernel writes one LoRA-down partial per RTQ_ACT_KQ columns (nhp of them).
struct FwdPlan {
  int64_t T, Tp, nhp;
  bool skinny;
  bool gemv;  // t <= 16 through rtq_gemv_* (see gemv_plan)
  size_t xq_bytes, xd_floats, xg_floats, h_floats, xdh_bytes;
  size_t dense_bytes;  // trainer-native weights: h
};

constexpr int kFwdWideTT = 4;     // rtq_fwd_*_w: 64 tokens x (16 * wide_rg) rows per workgroup
constexpr int kMmTile = 128;      // rtq_mm_*: 128 rows x 128 tokens per workgroup
// rtq_mm_* dynamic LDS: a 3-stage ring of half-chunk operands (codes, scales), reused after the
// K loop for the LoRA h and B rows of the tile (128 rows each, RTQ_LDS_RANK + 1 floats)
unsigned mm_lds_bytes(int type, int ttn, int ring) {  // ttn: token tiles of 16 per workgroup (8, 4 or 2)
  const unsigned stage =
      16u * (ttn * 2 * 64 + (type == RTQ_TYPE_Q4_0 ? 8 * 64 / 2 : 8 * 64) + 8 * 4 + 16 * std::max(ttn / 4, 1));
  return std::max((unsigned)ring * stage, (16u * ttn + 128u) * (RTQ_LDS_RANK + 1) * 4u);
}
// rtq_mmk*_* (K-quants, ttn 4 or 2): codes, sub-block scale words and activation codes per stage
unsigned mmk_lds_bytes(int type, int ttn, int ring) {
  const unsigned stage = 16u * (ttn * 2 * 64 + (type == RTQ_TYPE_Q4_K ? 8 * 64 / 2 : 8 * 64) + 8 * 4);
  return std::max((unsigned)ring * stage, (16u * ttn + 128u) * (RTQ_LDS_RANK + 1) * 4u);
}
// rtq_mmi8_* (ttn 4): int8 activation fragments, half the f16 ones' bytes
unsigned mmi8_lds_bytes(int type, int ttn, int ring) {
  const unsigned stage = 16u * (ttn * 64 + (type == RTQ_TYPE_Q4_0 ? 8 * 64 / 2 : 8 * 64) + 8 * 4 + 16 * (ttn / 4));
  return std::max((unsigned)ring * stage, (16u * ttn + 128u) * (RTQ_LDS_RANK + 1) * 4u);
}
constexpr int kFwdSkinnyRG = 4;   // rtq_fwd_*_s: 16 tokens x 64 rows per workgroup
int wide_rg(int type) { return is_kquant(type) ? 2 : 3; }
int gemv_rg(int type) { return byte_codes(type) ? 2 : 4; }
constexpr int64_t kGemvChunkLds = 4 * 64 * 16 + 4 * 2 * 16 * 4;  // LDS bytes per staged chunk
constexpr int64_t kGemvMaxChunks = 26;                          // <= 117 KB of staged activations

// GEMV grid: (row tiles of 4 waves x RG row groups, K splits); K is split across workgroups
// (atomics) until there are about two workgroups per CU and the staged chunks fit LDS, in whole
// chunks (two for K-quants)
struct GemvPlan {
  int64_t gx, gy, kcps;
};
GemvPlan gemv_plan(const rtq_ctx* c, const rtq_weight* w) {
  GemvPlan g;
  const int64_t Kc = w->Kp / 128, ngroups = w->Np / 16, rg = gemv_rg(w->type), unit = is_kquant(w->type) ? 2 : 1;
  g.gx = cdiv(ngroups, 4 * rg);
  int64_t ks = 1;
  if (g.gx < 2 * c->cu_count) ks = std::max<int64_t>(1, std::min<int64_t>(cdiv(2 * c->cu_count, g.gx), Kc / unit));
  ks = std::max(ks, cdiv(Kc, kGemvMaxChunks));
  g.kcps = roundup(cdiv(Kc, ks), unit);
  g.gy = cdiv(Kc, g.kcps);
  return g;
}

FwdPlan fwd_plan(const rtq_weight* w, int64_t t, int64_t r) {
  FwdPlan p{};
  p.T = t;
  if (is_dense(w->type)) {
    p.dense_bytes = (size_t)(t * std::max<int64_t>(r, 0)) * 4 + 2 * 256;
    return p;
  }
  p.skinny = t <= 16;
  p.gemv = p.skinny && r <= RTQ_LDS_RANK;
  // wide: 128-token padding, the token block of rtq_mm_* (rtq_fwd_*_w covers the first
  // cdiv(t, 64) token tiles of it)
  p.Tp = roundup(std::max<int64_t>(t, 1), p.skinny ? 16 : kMmTile);
  p.nhp = roundup(cdiv(w->Kp, RTQ_ACT_KQ), 4);
  p.xq_bytes = (size_t)p.Tp * w->Kp * 2;  // one f16 per element
  p.xd_floats = (size_t)(w->Kp / 32) * p.Tp;
  p.xdh_bytes = p.skinny ? 0 : p.xd_floats * 2;  // fp16 copy for rtq_mm_*
  p.xg_floats = p.gemv ? (size_t)(w->Kp / 32) * 2 * 16 : 0;
  p.h_floats = (size_t)p.nhp * t * std::max<int64_t>(r, 0);
  return p;
}

size_t fwd_ws_bytes(const FwdPlan& p) {
  return p.xq_bytes + p.xd_floats * 4 + p.xg_floats * 4 + p.h_floats * 4 + p.xdh_bytes + p.dense_bytes + 6 * 256;
}

// ------------------------------------------------------------------ trainer-native weights
// FrozenWeight::{F32, Q8_0} (src/frozen.rs:33-187) and the Linear LoRA math around them as f32
// products on the f32 MFMA GEMM of the decoder kernels (rtq_m_gemm*: exact f32 products, f32
// accumulation).  A TQ8_0 weight is read as codes plus one f32 scale per 32 and decoded in the
// GEMM's operand loads: no dequantised copy of the weight is materialised.

// C(m, n) (+)= sum_k A(m, k) B(k, n), A(m, k) = a_scale * A[m * sAm + k * sAk] (the product rounded
// first), B(k, n) = W[k * sBk + n * sBn] for f32 W, or the TQ8_0 weight w's decoded element at that
// index; C at row stride ldc.  64-row tiles when they fill the chip twice over, else 32-row tiles.
rtq_status dense_gemm(rtq_ctx* c, hipStream_t st, int64_t M, int64_t N, int64_t K, const float* A, int64_t sAm,
                      int64_t sAk, float a_scale, const float* B, const rtq_weight* q8, int64_t sBk, int64_t sBn,
                      float* C, int64_t ldc, bool acc) {
  if (M <= 0 || N <= 0) return RTQ_OK;
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) return fail(RTQ_ERR_INVALID, "f32 product too large");
  MGemmArgs ga{};
  ga.A = A;
  ga.B = q8 ? reinterpret_cast<const float*>(q8->wq) : B;
  ga.Bsc = q8 ? q8->wsc : nullptr;
  ga.C = C;
  ga.M = (int)M;
  ga.N = (int)N;
  ga.K = (int)K;
  ga.sAm = sAm;
  ga.sAk = sAk;
  ga.sBk = sBk;
  ga.sBn = sBn;
  ga.sCm = ldc;
  ga.sCn = 1;
  ga.divA = ga.divB = 1;
  ga.a_scale = a_scale;
  ga.accumulate = acc ? 1 : 0;
  ga.batch = 1;
  const int64_t tiles64 = cdiv(N, 64) * cdiv(M, 64);
  const int bm = tiles64 >= 2 * c->cu_count ? 64 : 32;
  const int64_t tiles = cdiv(N, 64) * cdiv(M, bm);
  if (tiles > INT32_MAX - 8) return fail(RTQ_ERR_INVALID, "f32 product too large");
  const int km = q8 ? (bm == 64 ? KM_GEMM_Q8 : KM_GEMM32_Q8) : (bm == 64 ? KM_GEMM : KM_GEMM32);
  return launch(c, K_MODEL + km, dim3((unsigned)roundup(tiles, 8)), dim3(256), st, ga);
}

// the weight as a B operand of y = x W^T (B(k, n) = W[n][k]) or dx = dy W (B(k, n) = W[k][n])
const float* dense_b(const rtq_weight* w) { return w->type == RTQ_TYPE_F32 ? reinterpret_cast<const float*>(w->wq) : nullptr; }
const rtq_weight* dense_q8(const rtq_weight* w) { return w->type == RTQ_TYPE_TQ8_0 ? w : nullptr; }

// y = x W^T (src/frozen.rs:121-122); + bias; + s (x A^T) B^T (src/linear.rs:73-93)
rtq_status enqueue_forward_dense(rtq_ctx* c, const rtq_weight* w, const float* x, int64_t t, float* y,
                                 const float* bias, const float* la, const float* lb, int64_t r, float s, Arena& ar,
                                 hipStream_t st) {
  const int64_t N = w->rows, K = w->cols;
  RTQ_TRY(dense_gemm(c, st, t, N, K, x, K, 1, 1.0f, dense_b(w), dense_q8(w), 1, K, y, N, false));
  if (bias) {
    DenseArgs da{nullptr, nullptr, nullptr, N, K, 0, t, y, bias, nullptr};
    RTQ_TRY(launch(c, K_DENSE_BIAS, dim3((unsigned)std::min<int64_t>(cdiv(t * N, 256), 8192)), dim3(256), st, da));
  }
  if (la && lb && r > 0) {
    float* hh = ar.take<float>((size_t)(t * r));
    if (ar.off > ar.cap) return fail(RTQ_ERR_INVALID, "internal: workspace too small");
    RTQ_TRY(dense_gemm(c, st, t, r, K, x, K, 1, 1.0f, la, nullptr, 1, K, hh, r, false));  // h = x A^T
    RTQ_TRY(dense_gemm(c, st, t, N, r, hh, r, 1, s, lb, nullptr, 1, r, y, N, true));     // y += (s h) B^T
  }
  return RTQ_OK;
}

// dx (+)= dy W (src/frozen.rs:139-167); with LoRA (src/linear.rs:97-121): h = x A^T,
// gb += (s dy)^T h, g = (s dy) B, ga += g^T x, dx += g A
rtq_status enqueue_backward_dense(rtq_ctx* c, const rtq_weight* w, const float* dy, int64_t t, float* dx,
                                  bool accumulate, const float* x, const float* la, const float* lb, int64_t r,
                                  float s, float* ga, float* gb, Arena& ar, hipStream_t st) {
  const int64_t N = w->rows, K = w->cols;
  RTQ_TRY(dense_gemm(c, st, t, K, N, dy, N, 1, 1.0f, dense_b(w), dense_q8(w), K, 1, dx, K, accumulate));
  if (la && lb && r > 0) {
    float* hh = ar.take<float>((size_t)(t * r));
    float* g = ar.take<float>((size_t)(t * r));
    if (ar.off > ar.cap) return fail(RTQ_ERR_INVALID, "internal: workspace too small");
    RTQ_TRY(dense_gemm(c, st, t, r, K, x, K, 1, 1.0f, la, nullptr, 1, K, hh, r, false));  // h = x A^T
    RTQ_TRY(dense_gemm(c, st, N, r, t, dy, 1, N, s, hh, nullptr, r, 1, gb, r, true));     // gb += (s dy)^T h
    RTQ_TRY(dense_gemm(c, st, t, r, N, dy, N, 1, s, lb, nullptr, r, 1, g, r, false));     // g = (s dy) B
    RTQ_TRY(dense_gemm(c, st, r, K, t, g, 1, r, 1.0f, x, nullptr, K, 1, ga, K, true));    // ga += g^T x
    RTQ_TRY(dense_gemm(c, st, t, K, r, g, r, 1, 1.0f, la, nullptr, K, 1, dx, K, true));   // dx += g A
  }
  return RTQ_OK;
}

// ------------------------------------------------------------------ enqueue: forward
// y = x.W^T (+bias) (+ s h.B^T);  isums (debug) receives the per-block integer sums.
// hp_keep (optional, nhp * t * r floats): the LoRA-down partials go there instead of the workspace,
// for a later enqueue_backward of the same x to reuse
// sw_g / sw_u (optional, quantised weights): x is SwiGLU's silu(g) * u (rows of stride sw_ld), formed
// by the activation kernel and written to x
struct SwiGluIn {
  const float* g;
  const float* u;
  int64_t ld;
};
rtq_status enqueue_forward(rtq_ctx* c, const rtq_weight* w, const float* x, int64_t t, float* y, const float* bias,
                           const float* la, const float* lb, int64_t r, float s, int32_t* isums, Arena& ar,
                           hipStream_t st, float* hp_keep = nullptr, const RankBlocks* rb = nullptr,
                           const SwiGluIn* sw = nullptr, const NormIn* nf = nullptr) {
  if (t <= 0) return RTQ_OK;
  const bool lora = la && lb && r > 0;
  const RankBlocks rbv = lora && rb ? *rb : RankBlocks{};
  if (is_dense(w->type)) {
    if (sw || nf) return fail(RTQ_ERR_UNSUPPORTED, "internal: SwiGLU / norm input of a dense weight");
    return enqueue_forward_dense(c, w, x, t, y, bias, la, lb, lora ? r : 0, s, ar, st);
  }
  // the activation kernel's inputs: x, or SwiGLU's g / u, or RMSNorm's a (+ b) (x then an output)
  auto act_in = [&](ActArgs& aa) {
    if (sw) {
      aa.sg = sw->g;
      aa.su = sw->u;
      aa.ldsg = (int)sw->ld;
    }
    if (nf) {
      aa.na = nf->a;
      aa.nb = nf->b;
      aa.nh = nf->h;
      aa.nw = nf->w;
      aa.ninv = nf->inv;
      aa.neps = nf->eps;
      aa.noff = nf->off;
    }
  };
  // t <= 4: one launch that quantises x itself (codes, scales and h in LDS, at most 64 KB)
  // (not where a later backward reads the LoRA-down partials: this kernel keeps none; not with an
  // adapter: every workgroup would form h = x A^T again, and the small adapted shapes are faster on
  // the activation kernel's partials - q_proj 2048 x 1024 at t = 1: 33 against 12 us)
  if (c->gemvq && t <= 4 && !isums && !sw && !nf && !hp_keep && !lora) {
    const int nt = t == 1 ? 1 : 4;
    const size_t lds = (size_t)nt * w->Kp + (size_t)nt * (w->Kp / 32) * 4 * (w->type == RTQ_TYPE_Q4_0 ? 5 : 2) +
                       (size_t)nt * RTQ_LDS_RANK * 4;
    if (lds <= 65536) {
      const int rg = byte_codes(w->type) ? RTQ_GQ_RG8 : RTQ_GQ_RG4;
      const int64_t ntiles = cdiv(w->Np / 16, rg);
      // waves per CU: 24 for the nibble layouts (their VGPRs allow 20 - 24 resident), 8 for Q6_K and 4
      // for Q8_0 (longer streams per wave; LM head at t = 1, one MI355X: Q4_0 21.1 us at 24 against
      // 23.4 at 16, Q4_K 24.8 against 26.7, Q6_K 34.4 at 8 against 36.8 at 6 and 37.4 at 10, Q8_0
      // 30.7 at 4 against 31.9 at 8: 238 workgroups, one per CU, where 5 or 6 give some CUs two,
      // 38.5 / 35.5 us); every wave takes the same number of tiles (the last ones fewer)
      const int64_t wpc = c->gemvq_wpc > 0 ? c->gemvq_wpc
                                            : (w->type == RTQ_TYPE_Q8_0 ? 4 : byte_codes(w->type) ? 8 : 24);
      const int64_t maxw = (int64_t)c->cu_count * wpc, per = cdiv(ntiles, maxw), nwaves = cdiv(ntiles, per);
      GemvqArgs ga{w->wq, w->wdr, w->wsb, (int)w->Np, (int)w->Kp, x, (int)t, (int)w->rows, (int)w->cols, y, bias,
                   lora ? la : nullptr, lb, lora ? (int)r : 0, s, rbv, (int)ntiles, (int)per};
      set_work(c, w, t, lora ? r : 0, false);
      return launch(c, (nt == 1 ? K_GEMVQ1 : K_GEMVQ4) + fmt_index(w->type), dim3((unsigned)cdiv(nwaves, 4)),
                    dim3(256), st, ga, (unsigned)lds);
    }
  }
  FwdPlan p = fwd_plan(w, t, lora ? r : 0);
  // the debug sums come from the skinny / wide kernels; the GEMV pays off once its row tiles alone
  // give a workgroup per CU (an LM head), below that the skinny kernel's K split wins
  if (isums || cdiv(w->Np / 16, 4 * gemv_rg(w->type)) < c->cu_count) p.gemv = false;
  void* xq = ar.take<char>(p.xq_bytes);
  float* xd = ar.take<float>(p.xd_floats);
  float* xg = p.gemv ? ar.take<float>(p.xg_floats) : nullptr;
  float* hp = lora ? (hp_keep ? hp_keep : ar.take<float>(p.h_floats)) : nullptr;
  if (ar.off > ar.cap) return fail(RTQ_ERR_INVALID, "internal: workspace too small");
  if (p.gemv) {
    const GemvPlan gp = gemv_plan(c, w);
    const float gbias = w->type == RTQ_TYPE_Q4_0 ? 1032.0f : (w->type == RTQ_TYPE_Q8_0 ? 1152.0f : 0.0f);
    ActArgs aa{x, (int)t, (int)w->cols, (int)p.Tp, (int)w->Kp, xq, xd, xg, gbias, lora ? la : nullptr, (int)r, hp,
               gp.gy > 1 ? y : nullptr, (int)w->rows, nullptr};
    act_in(aa);
    RTQ_TRY(launch(c, is_kquant(w->type) ? K_ACT_PREP_K : K_ACT_PREP, dim3((unsigned)(p.Tp / 16), (unsigned)p.nhp),
                   dim3(256), st, aa));
    FwdArgs fa{};
    fa.wq = w->wq;
    fa.wd = w->wd;
    fa.wdr = w->wdr;
    fa.xg = xg;
    fa.wsb = w->wsb;
    fa.Np = (int)w->Np;
    fa.Kp = (int)w->Kp;
    fa.xq = xq;
    fa.xd = xd;
    fa.Tp = (int)p.Tp;
    fa.T = (int)t;
    fa.N = (int)w->rows;
    fa.K = (int)w->cols;
    fa.kc_per_split = (int)gp.kcps;
    fa.y = y;
    fa.bias = bias;
    fa.hp = hp;
    fa.nhp = (int)p.nhp;
    fa.lb = lb;
    fa.r = (int)r;
    fa.s = s;
    fa.rb = rbv;
    const int kid = K_GEMV + fmt_index(w->type);
    set_work(c, w, t, lora ? r : 0, false);
    return launch(c, kid, dim3((unsigned)gp.gx, (unsigned)gp.gy), dim3(256), st, fa,
                  (unsigned)(gp.kcps * kGemvChunkLds));
  }
  const int64_t Kc = w->Kp / 128;
  const bool kq = is_kquant(w->type);
  const bool w8 = !p.skinny && !isums && !kq && c->fwd_waves == 8;  // rtq_fwd_*_w8[r2]
  const int64_t gy = p.skinny ? p.Tp / 16 : cdiv(t, 16 * kFwdWideTT);
  // the eight-wave forward with 32-row tiles wherever 48-row tiles would leave CUs without a
  // workgroup, 16-row tiles wherever 32-row ones still would (RTQ_FWD_RG: 1, 2 or 3 forces one).
  // Measured at 256 tokens (one MI355X, per forward call): kv_proj 1024 x 1024 24.8 -> 20.3 us,
  // down_proj 1024 x 3072 32.7 -> 24.4 at 32 rows (both still split K)
  int wrg = 3;
  if (w8) {
    if (c->fwd_rg >= 1 && c->fwd_rg <= 3) wrg = c->fwd_rg;
    else if (cdiv(w->Np / 16, 3) * gy < c->cu_count) wrg = cdiv(w->Np / 16, 2) * gy < c->cu_count ? 1 : 2;
  }
  const int64_t rg_per_wg = p.skinny ? kFwdSkinnyRG : (w8 ? wrg : wide_rg(w->type));
  const int64_t gx = cdiv(w->Np / 16, rg_per_wg);
  // the large-grid kernel once its 128 x 128 tiles alone give a workgroup per CU, else its
  // 128 x 64 tiles if those do
  const int64_t mm_rows = cdiv(w->Np / 16, 8);
  const int64_t mm128 = mm_rows * (p.Tp / kMmTile), mm64 = mm_rows * (p.Tp / 64), mm32 = mm_rows * (p.Tp / 32);
  int mm_ttn = 0;  // token tiles per workgroup of the chosen rtq_mm kernel, 0: none
  if (!p.skinny && !isums && !is_kquant(w->type)) {
    if (c->fwd_mm == 1) mm_ttn = 8;
    else if (c->fwd_mm == 2) mm_ttn = 4;
    else if (c->fwd_mm == 3) mm_ttn = 2;
    // automatic: 128-token tiles when they give every CU a workgroup; else 32-token tiles when 64-token
    // ones would (two or more workgroups per CU hide the K loop's latencies better than one: 1.15
    // against 1.27 ms per Qwen3-0.6B-shaped 512-token step over its q|k|v and gate|up products)
    else if (c->fwd_mm < 0) mm_ttn = mm128 >= c->cu_count ? 8 : (mm64 >= c->cu_count ? 2 : 0);
  }
  const bool mm = mm_ttn > 0;
  // the int8-MFMA kernel where the 128- or 64-token tiles are chosen, on 64-token tiles (its 128-token
  // form holds 300 VGPRs, one wave per SIMD).  Automatic: for Q8_0 weights, whose codes reach the
  // i8 MFMA as they lie in LDS; measured per forward call (activation kernel included) at 2048
  // tokens: LM head 151936 x 1024 980 against 1020 us (f16, 128-token tiles), 28672 x 4096 848
  // against 897, 6144 x 4096 241 against 259 (f16, 64-token tiles); Q4_0 mixed (1043 against
  // 1005 us on the LM head, 864 against 906 on 28672 x 4096), so Q4_0 keeps the f16 kernels.
  // Both agree bit for bit without an adapter.
  const bool mmi8 = mm && (mm_ttn == 8 || mm_ttn == 4) &&
                    (c->fwd_i8 == 1 || (c->fwd_i8 < 0 && w->type == RTQ_TYPE_Q8_0));
  if (mmi8) mm_ttn = 4;
  // K-quants: the LDS-ring kernel on 64-token tiles where they give every CU a workgroup, else on
  // 32-token tiles where those do.  Measured per forward call at 2048 tokens against the tile
  // kernel (rtq_fwd_*_w): Qwen3-4B q | k | v 226 -> 179 us, gate | up 641 -> 464, down (Q6_K) 384
  // -> 323, LM head Q4_K 1778 -> 1307 (32-token tiles: 214, 585, 375, 1673)
  int mmk_ttn = 0;
  if (!p.skinny && !isums && is_kquant(w->type)) {
    if (c->fwd_mmk == 1) mmk_ttn = 4;
    else if (c->fwd_mmk == 2) mmk_ttn = 2;
    else if (c->fwd_mmk < 0) mmk_ttn = mm64 >= c->cu_count ? 4 : (mm32 >= c->cu_count ? 2 : 0);
  }
  const int64_t mm_tiles = mm_ttn == 8 ? mm128 : mm_ttn == 4 ? mm64 : mm32;
  // split K across workgroups when the output alone gives too few of them (atomics into a
  // zeroed y); every split keeps at least one half chunk per wave (K-quants: one super-block of
  // two chunks per wave, and splits on super-block boundaries).  The eight-wave tiles never split
  // K (smaller row tiles fill the CUs instead): each output is then summed by one workgroup in one
  // order whatever the token count, so a packed batch and its examples, run at other token counts,
  // get the same bits
  const int64_t tiles = gx * gy;
  int64_t ks = 1;
  if (!isums && !mm && !mmk_ttn && !w8 && tiles < c->cu_count) {
    const int64_t want = cdiv(p.skinny ? 2 * c->cu_count : c->cu_count, tiles);
    ks = std::max<int64_t>(1, std::min<int64_t>(want, Kc / (kq ? 8 : 2)));
  }
  int64_t kcps = cdiv(Kc, ks);
  if (kq) kcps = roundup(kcps, 2);
  ks = cdiv(Kc, kcps);

  uint16_t* xdh = mm ? ar.take<uint16_t>(p.xdh_bytes / 2) : nullptr;
  if (ar.off > ar.cap) return fail(RTQ_ERR_INVALID, "internal: workspace too small");
  ActArgs aa{x, (int)t, (int)w->cols, (int)p.Tp, (int)w->Kp, xq, xd, nullptr, 0.0f, lora ? la : nullptr, (int)r, hp,
             ks > 1 ? y : nullptr, (int)w->rows, xdh};
  act_in(aa);
  aa.xq_i8 = mmi8 ? 1 : 0;
  // the block norms' activations (Q8_0 f16 fragments) on 8-token tiles: twice the workgroups, each
  // reading half the rows whole for the sums of squares (the same bits as the 16-token kernel)
  const int att = c->act_tt < 16 && nf && !kq && !mmi8 && !aa.zero_y && !aa.sg && !aa.xg ? c->act_tt : 16;
  RTQ_TRY(launch(c, att == 8 ? K_ACT_PREP8 : att == 4 ? K_ACT_PREP4 : kq ? K_ACT_PREP_K : K_ACT_PREP,
                 dim3((unsigned)(p.Tp / att), (unsigned)p.nhp), dim3(256), st, aa));
  FwdArgs fa{};
  fa.wq = w->wq;
  fa.wd = w->wd;
  fa.wdr = w->wdr;  // rtq_mm_* reads the row-major scales
  fa.wsb = w->wsb;
  fa.Np = (int)w->Np;
  fa.Kp = (int)w->Kp;
  fa.xq = xq;
  fa.xd = xd;
  fa.Tp = (int)p.Tp;
  fa.T = (int)t;
  fa.N = (int)w->rows;
  fa.K = (int)w->cols;
  fa.kc_per_split = (int)kcps;
  fa.y = y;
  fa.bias = bias;
  fa.hp = hp;
  fa.nhp = (int)p.nhp;
  fa.lb = lb;
  fa.r = (int)r;
  fa.s = s;
  fa.rb = rbv;
  fa.isums = isums;
  fa.xdh = xdh;
  if (mm && (!fa.wq || !fa.wdr || !fa.xq || !fa.xdh || !fa.y))
    return fail(RTQ_ERR_INVALID, "internal: rtq_mm_* operand missing");
  set_work(c, w, t, lora ? r : 0, false);
  if (mmi8)
    return launch(c, K_MMI8_64_Q4_0 + (w->type == RTQ_TYPE_Q4_0 ? 0 : 1), dim3((unsigned)mm_tiles), dim3(256), st, fa,
                  mmi8_lds_bytes(w->type, 4, RTQ_MM64_RING));
  if (mmk_ttn) {
    if (!fa.wq || !fa.wd || !fa.wsb || !fa.xq || !fa.xd || !fa.y)
      return fail(RTQ_ERR_INVALID, "internal: rtq_mmk_* operand missing");
    const int kid = (mmk_ttn == 4 ? K_MMK64_Q4_K : K_MMK32_Q4_K) + (w->type == RTQ_TYPE_Q4_K ? 0 : 1);
    return launch(c, kid, dim3((unsigned)(mmk_ttn == 4 ? mm64 : mm32)), dim3(256), st, fa,
                  mmk_lds_bytes(w->type, mmk_ttn, mmk_ttn == 4 ? RTQ_MM64_RING : RTQ_MM32_RING));
  }
  if (mm) {
    const int ring = mm_ttn == 8 ? RTQ_MM_RING : mm_ttn == 4 ? RTQ_MM64_RING : RTQ_MM32_RING;
    return launch(c, (mm_ttn == 8 ? K_MM_Q4_0 : mm_ttn == 4 ? K_MM64_Q4_0 : K_MM32_Q4_0) + (w->type == RTQ_TYPE_Q4_0 ? 0 : 1),
                  dim3((unsigned)mm_tiles), dim3(256), st, fa, mm_lds_bytes(w->type, mm_ttn, ring));
  }
  int kid = (p.skinny ? (isums ? K_FWD_S_ISUMS : K_FWD_S) : (isums ? K_FWD_W_ISUMS : K_FWD_W)) + fmt_index(w->type);
  int threads = 256;
  if (w8) {
    kid = (wrg == 1 ? K_FWD_Q4_0_W8R1 : wrg == 2 ? K_FWD_Q4_0_W8R2 : K_FWD_Q4_0_W8) + (w->type == RTQ_TYPE_Q4_0 ? 0 : 1);
    threads = 512;
  }
  return launch(c, kid, dim3((unsigned)gx, (unsigned)gy, (unsigned)ks), dim3(threads), st, fa);
}

// ------------------------------------------------------------------ enqueue: backward
// dx split plan.
//   t > 16 (rtq_dx_*): K chunks x 64-token tiles x row splits, about one 8-wave workgroup per CU
//     (more splits add partial-sum traffic: each split writes and the finish kernel reads a
//     64-token-padded T x K block);
//   t <= 16 (rtq_dx16_*): K chunks x row splits, about two 4-wave workgroups per CU with at least
//     four 32-row steps each (partials are T x K floats per split; LM head 151936 x 1024 at T = 16,
//     one backward call, 64 against 96 splits: Q4_0 58.7 / 62.4 us, Q8_0 64.1 / 65.9, Q4_K 72.7 /
//     73.7, Q6_K 75.1 / 76.1);
//   rtq_dxw_*: as the first, with 256-token tiles, where that grid fills the CUs (see dx_plan).
struct DxPlan {
  int64_t splits, nps;
  bool tok16;
  bool wide;  // rtq_dxw_*: 256-token tiles (each dequantised weight element feeds 4x the MFMAs)
  bool t32;   // rtq_dx32_*: 32-token tiles on four-wave workgroups (same partial layout as rtq_dx_*)
  bool v1;    // rtq_dxv1_*: t == 1 on f32 FMAs (partials as rtq_dx16_*)
  size_t part_floats;
};
DxPlan dx_plan(const rtq_ctx* c, const rtq_weight* w, int64_t t) {
  DxPlan p;
  p.tok16 = t <= 16;
  const int64_t Kc = w->Kp / 128, steps = w->Np / 32;
  // 256-token tiles when their grid fills whole rounds of the CUs (at least 85%) with at least 16
  // row steps per workgroup; the split count rounds to the nearest whole grid (up to 32 splits)
  const int64_t per_split = Kc * cdiv(t, 256);
  const int64_t wsplits = std::max<int64_t>(1, std::min<int64_t>(std::min<int64_t>(32, steps),
                                                                  (c->cu_count + per_split / 2) / per_split));
  const int64_t wgrid = roundup(cdiv(t, 256) * wsplits, 8) * Kc;
  const bool wide_fits = 100 * wgrid >= 85 * cdiv(wgrid, c->cu_count) * c->cu_count && steps / wsplits >= 16;
  p.wide = !p.tok16 && (c->dx_wide == 1 || (c->dx_wide < 0 && wide_fits));
  p.t32 = !p.tok16 && !p.wide && c->dx_32 > 0;
  int64_t splits;
  if (p.tok16)
    splits = std::max<int64_t>(1, std::min<int64_t>(std::min<int64_t>(std::max<int64_t>(steps / 4, 1), 256),
                                                    cdiv(2 * c->cu_count, Kc)));
  else if (p.wide)
    splits = wsplits;
  else
    splits = std::max<int64_t>(1, std::min<int64_t>(std::min<int64_t>(steps, 16),
                                                    cdiv(c->dx_wpc * c->cu_count, Kc * cdiv(t, 64))));
  if (p.t32 && c->dx_32 == 2) splits = std::max<int64_t>(1, splits / 2);
  if (c->dx_splits > 0)
    splits = std::min<int64_t>(std::min<int64_t>(steps, p.tok16 ? 256 : (p.wide ? 64 : 16)), c->dx_splits);
  p.nps = cdiv(steps, splits) * 32;
  p.v1 = t == 1 && c->dxv && (uint64_t)(w->Np / 16) * (w->Kp / 128) * 2048u < (1ull << 32);
  // rtq_dxv1_*: about three four-wave workgroups per CU, each split at least 8 row groups of 16.
  // Measured on the LM head (151936 x 1024) at t = 1, one backward call, two, three, four, six
  // workgroups per CU: Q4_0 24.4 / 24.7 / 25.0 / 25.9 us, Q4_K 27.6 / 27.3 / 27.9 / 29.6, Q6_K
  // 37.7 / 36.3 / 36.5 / 37.5, Q8_0 36.6 / 34.9 / 35.6 / 35.9
  if (p.v1) {
    const int64_t ngr = w->Np / 16;
    const int64_t sv = std::max<int64_t>(1, std::min<int64_t>(cdiv(c->dxv_wpc * c->cu_count, Kc), cdiv(ngr, 8)));
    p.nps = cdiv(ngr, sv) * 16;
  }
  p.splits = cdiv(w->Np, p.nps);
  p.part_floats = p.tok16 ? (size_t)(p.splits * t * w->cols) : (size_t)(p.splits * roundup(t, 64) * w->Kp);
  return p;
}

// partial-product slices of the LoRA reductions over n columns (multiple of 4, see sum_partials)
int64_t lora_slices(int64_t n) { return roundup(cdiv(std::max<int64_t>(n, 1), RTQ_ACT_KQ), 4); }

// backward workspace: h, g [t x r], their slice partials [t][r][slices], dx split partials
size_t bwd_ws_bytes(const rtq_ctx* c, const rtq_weight* w, int64_t t, int64_t r) {
  const int64_t n = w->rows, k = w->cols;
  if (is_dense(w->type)) return (size_t)(2 * t * std::max<int64_t>(r, 0)) * 4 + 3 * 256;
  const int64_t sl = roundup(cdiv(std::max<int64_t>(n, 1), RTQ_ACT_KQ), 4) + roundup(cdiv(std::max<int64_t>(k, 1), RTQ_ACT_KQ), 4);
  return (size_t)((2 + sl) * t * std::max<int64_t>(r, 0)) * 4 + dx_plan(c, w, std::max<int64_t>(t, 1)).part_floats * 4 +
         (size_t)(lora_slices(n) * t) * 4 + 7 * 256;
}


// dx (+)= dy.W (accumulate: FrozenMatmul::backward_input; otherwise dx is overwritten, as
// Linear::backward returns a fresh dx); with LoRA also dx += g.A, ga += g^T x, gb += (s dy)^T h
// (g = s dy.B, h = x.A^T).  Kernels: [rtq_bwd_prep: slice partials of h, g] -> rtq_dx_* (per-split
// partials of dx; its last grid row sums the h, g partials) -> rtq_bwd_finish.
// defer (or null): the dA / dB tiles are not launched but described in defer->job, with h and g in
// defer->h / defer->g (rtq_linear_backward_defer_d)
struct LoraDefer {
  float* h;
  float* g;
  LoraGradArgs* job;
  const SwiGluBwd* sw;  // or null: the finish applies SwiGLU's backward to dx instead of storing it
};
rtq_status enqueue_backward(rtq_ctx* c, const rtq_weight* w, const float* dy, int64_t t, float* dx, bool accumulate,
                            const float* x, const float* la, const float* lb, int64_t r, float s, float* ga,
                            float* gb, Arena& ar, hipStream_t st, const RankBlocks* rb = nullptr,
                            const float* hp_have = nullptr, const LoraDefer* defer = nullptr) {
  if (t <= 0) return RTQ_OK;
  const bool lora = la && lb && r > 0;
  if (is_dense(w->type))
    return enqueue_backward_dense(c, w, dy, t, dx, accumulate, x, la, lb, lora ? r : 0, s, ga, gb, ar, st);
  const int N = (int)w->rows, K = (int)w->cols;
  if ((uint64_t)t * (uint64_t)N * 4u >= (1ull << 31))
    return fail(RTQ_ERR_INVALID, "dy of %lld x %d floats exceeds the 2 GiB buffer-offset range", (long long)t, N);
  const DxPlan dp = dx_plan(c, w, t);
  const int64_t nhq = lora_slices(K), ngq = lora_slices(N);
  if (defer && defer->job) defer->job->n_gb = defer->job->n_ga = 0;
  if (!lora) defer = nullptr;
  float* h = lora ? (defer ? defer->h : ar.take<float>((size_t)(t * r))) : nullptr;
  float* g = lora ? (defer ? defer->g : ar.take<float>((size_t)(t * r))) : nullptr;
  // hp_have: the forward's LoRA-down partials of this x (same slices), so only g is computed here
  const bool have_h = lora && hp_have != nullptr;
  float* hp = lora ? (have_h ? const_cast<float*>(hp_have) : ar.take<float>((size_t)(nhq * t * r))) : nullptr;
  float* gp = lora ? ar.take<float>((size_t)(ngq * t * r)) : nullptr;
  float* part = ar.take<float>(dp.part_floats);
  // row maxima of dy per 256-row slice, for the f16 range of rtq_dx_* / rtq_dxw_* (from the LoRA g
  // partial kernel, or the same kernel with no adapter)
  float* dymax = dp.tok16 ? nullptr : ar.take<float>((size_t)(ngq * t));
  if (ar.off > ar.cap) return fail(RTQ_ERR_INVALID, "internal: workspace too small");
  if (lora) {
    // h partials: 16 tokens per workgroup; g partials: 64 where those workgroups alone give every
    // CU one; else 32 where those give at least half of the CUs one and no CU two (the 32-token
    // form splits each slice's rows over two waves, so twice the workgroups run half the MFMA
    // chain); else 64 where those give at least half of the CUs one; else 16.  Measured per
    // configs[2] call (512 tokens): q|k|v (16 slices, r 48) 8.33 -> 7.46 us at 32; gate|up (24
    // slices, r 32, 384 workgroups at 32) 8.53 -> 9.41, so 64 there
    const int64_t g64 = c->g64_min >= 0 ? c->g64_min : c->cu_count / 2, n64 = cdiv(t, 64) * ngq, n32 = cdiv(t, 32) * ngq;
    int gtok = n64 >= std::max<int64_t>(g64, c->cu_count) ? 64 : (n32 >= g64 && n32 <= c->cu_count) ? 32 : n64 >= g64 ? 64 : 16;
    if (c->gtok == 16 || c->gtok == 32 || c->gtok == 64) gtok = c->gtok;
    BwdPrepArgs pa{x, la, K, dy, lb, N, (int)t, (int)r, hp, (int)nhq, gp, (int)ngq, dymax, RankBlocks{},
                   have_h ? (int)nhq : 0, gtok};
    if (rb) pa.rb = *rb;
    RTQ_TRY(launch(c, K_BWD_PREP, dim3((unsigned)cdiv(t, have_h ? gtok : 16), (unsigned)(have_h ? ngq : nhq + ngq)),
                   dim3(256), st, pa));
  } else if (dymax) {
    const int gtok = cdiv(t, 64) * ngq >= (c->g64_min >= 0 ? c->g64_min : c->cu_count / 2) ? 64 : 16;
    BwdPrepArgs pa{nullptr, nullptr, K, dy, nullptr, N, (int)t, 0, nullptr, 0, nullptr, (int)ngq, dymax, RankBlocks{},
                   0, gtok};
    RTQ_TRY(launch(c, K_BWD_PREP, dim3((unsigned)cdiv(t, gtok), (unsigned)ngq), dim3(256), st, pa));
  }
  DxArgs xa{w->wq, w->wd, w->wsb, (int)w->Np, (int)w->Kp, dy, (int)t, N, K, (int)dp.nps, (int)dp.splits, part,
            lora ? hp : nullptr, lora ? gp : nullptr, (int)nhq, (int)ngq, (int)r, s, h, g, dymax, (int)ngq,
            w->dx_wsc, w->dx_wunsc, w->wdr};
  const int kid = (dp.v1 ? K_DXV1 : dp.tok16 ? K_DX16 : (dp.wide ? K_DXW : (dp.t32 ? K_DX32 : K_DX))) + fmt_index(w->type);
  set_work(c, w, t, 0, true);
  // t > 16: (token group, split) units of K-chunk workgroups, padded to a multiple of 8 (XCD order)
  const int64_t nmain = dp.tok16 ? (w->Kp / 128) * dp.splits
                                 : roundup(cdiv(t, dp.wide ? 256 : (dp.t32 ? 32 : 64)) * dp.splits, 8) * (w->Kp / 128);
  const int64_t nfin = lora ? std::min<int64_t>(64, cdiv(t * r, 512)) : 0;  // LoRA finalisers
  RTQ_TRY(launch(c, kid, dim3((unsigned)(nmain + nfin)), dim3(dp.tok16 || dp.t32 ? 256 : 512), st, xa));
  const int64_t jt = cdiv(r, 16);
  LoraGradArgs fa{dy, h, g, x, la, (int)t, N, K, (int)r, s, gb, ga, dx, 0, 0, 0, part, (int)dp.splits, accumulate ? 1 : 0,
                  dp.tok16 ? 1 : 0, RankBlocks{}};
  if (rb) fa.rb = *rb;  // block-diagonal adapter: dB tiles outside every member's block exit at once
  // dB / dA: one workgroup per 64-row x 16-rank tile; dx: one wave per quarter of a dx fragment (or
  // per token and 64 columns); nw waves per workgroup, 16 when the dA / dB tiles reduce over many tokens
  fa.n_gb = lora ? (int)(cdiv(N, 64) * jt) : 0;
  fa.n_ga = lora ? (int)(cdiv(K, 64) * jt) : 0;
  const int nw = lora && t >= 256 ? 16 : 4;
  fa.n_dx = dp.tok16 ? (int)cdiv(t * cdiv(K, 64), nw) : (int)cdiv((w->Kp / 128) * cdiv(t, 64) * 32, nw);
  // dx alone: row-major partials of more than 16 splits take a workgroup per (token, 64 columns)
  const bool wide_rows = dp.tok16 && dp.splits > 16;
  const Kid kdx = dp.splits <= 4 ? K_BWD_FINISH_DX : wide_rows ? K_BWD_FINISH_ROWS : K_BWD_FINISH;
  const unsigned gdx = wide_rows ? (unsigned)(t * cdiv(K, 64)) : 0;
  if (defer) {  // dA / dB later, in a batch; here the dx partials (+ g.A) alone, 4 waves per workgroup
    *defer->job = fa;
    defer->job->n_dx = 0;
    defer->job->part = nullptr;
    fa.n_gb = fa.n_ga = 0;
    fa.n_dx = dp.tok16 ? (int)cdiv(t * cdiv(K, 64), 4) : (int)cdiv((w->Kp / 128) * cdiv(t, 64) * 32, 4);
    if (defer->sw) {
      fa.swg = defer->sw->g;
      fa.swu = defer->sw->u;
      fa.swdg = defer->sw->dg;
      fa.swdu = defer->sw->du;
      fa.swld = defer->sw->ld;
      fa.sw_keep = defer->sw->keep_dh ? 1 : 0;
    }
    return launch(c, kdx, dim3(wide_rows ? gdx : (unsigned)fa.n_dx), dim3(256), st, fa);
  }
  if (!lora) return launch(c, kdx, dim3(wide_rows ? gdx : (unsigned)fa.n_dx), dim3(256), st, fa);
  return launch(c, nw == 16 ? K_BWD_FINISH16 : K_BWD_FINISH, dim3((unsigned)(fa.n_gb + fa.n_ga + fa.n_dx)),
                dim3(64 * nw), st, fa);
}

void set_work(rtq_ctx* c, const rtq_weight* w, int64_t t, int64_t r, bool backward) {
  const double N = (double)w->rows, K = (double)w->cols, T = (double)t, R = (double)std::max<int64_t>(r, 0);
  const double wb = (double)w->gguf_bytes;
  if (backward) {
    c->next_flops = 2.0 * T * N * K;
    c->next_bytes = wb + 4.0 * T * (N + K);
  } else {
    c->next_flops = 2.0 * T * N * K + 2.0 * T * R * (K + N);
    c->next_bytes = wb + 4.0 * T * (N + K) + 4.0 * R * (K + N);
  }
}

rtq_status check_weight(rtq_ctx* c, const rtq_weight* w) {
  if (!c) return fail(RTQ_ERR_INVALID, "null context");
  if (!w) return fail(RTQ_ERR_INVALID, "null weight");
  if (w->ctx != c) return fail(RTQ_ERR_INVALID, "weight belongs to another context");
  return RTQ_OK;
}

rtq_status check_lora(const rtq_lora* l, bool* on, int64_t* r, float* s) {
  *on = false;
  *r = 0;
  *s = 0.0f;
  if (!l || !l->enabled || l->rank <= 0) return RTQ_OK;
  if (!l->a || !l->b) return fail(RTQ_ERR_INVALID, "lora enabled with null a/b");
  if (l->rank > 4096) return fail(RTQ_ERR_INVALID, "lora rank %lld too large", (long long)l->rank);
  *on = true;
  *r = l->rank;
  *s = l->alpha / (float)l->rank;  // Lora::scale, src/linear.rs:26-28
  return RTQ_OK;
}

rtq_status check_t(int64_t t) {
  if (t < 0) return fail(RTQ_ERR_INVALID, "negative token count");
  if (t > (1LL << 24)) return fail(RTQ_ERR_INVALID, "token count %lld too large", (long long)t);
  return RTQ_OK;
}

// ------------------------------------------------------------------ weight repack (host)
// GGUF blocks -> fragment layout (see rtq_kargs.h).  Padding rows/blocks get scale 0 and
// zero-valued codes.

// Places the codes of block j of chunk kc, row li of row group rg.  Nibble layouts take 16 bytes
// (element e in the low nibble of byte e, element e + 16 in its high nibble), byte layouts 32.
void place_codes(bool bytes, const uint8_t* codes, int64_t rg, int64_t kc, int64_t li, int64_t j, int64_t Kc,
                 uint8_t* wq) {
  if (!bytes) {
    for (int g = 0; g < 4; g++) memcpy(wq + ((rg * Kc + kc) * 64 + li + 16 * g) * 16 + j * 4, codes + 4 * g, 4);
    return;
  }
  const int64_t part = j / 2, off = (j % 2) * 8;
  for (int g = 0; g < 4; g++) {
    uint8_t* dst = wq + (((rg * Kc + kc) * 2 + part) * 64 + li + 16 * g) * 16 + off;
    memcpy(dst, codes + 4 * g, 4);
    memcpy(dst + 4, codes + 16 + 4 * g, 4);
  }
}

inline uint16_t le16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

void repack_q32(int type, const uint8_t* src, int64_t N, int64_t K, int64_t Np, int64_t Kp, uint8_t* wq,
                uint16_t* wd, uint16_t* wdr) {
  const int64_t Kc = Kp / 128, nb = K / 32, nbp = Kp / 32, bb = block_bytes(type), rb = nb * bb;
  const bool q4 = type == RTQ_TYPE_Q4_0;
  for (int64_t n = 0; n < Np; n++) {
    const int64_t rg = n / 16, li = n % 16;
    for (int64_t b = 0; b < nbp; b++) {
      const int64_t kc = b / 4, j = b % 4;
      uint16_t d = 0;
      uint8_t codes[32];
      if (n < N && b < nb) {
        const uint8_t* blk = src + n * rb + b * bb;
        d = le16(blk);
        memcpy(codes, blk + 2, q4 ? 16 : 32);
      } else {
        memset(codes, q4 ? 0x88 : 0, 32);  // code value 0
      }
      place_codes(!q4, codes, rg, kc, li, j, Kc, wq);
      wd[RTQ_WD_INDEX(rg, kc, Kc, li, j)] = d;
      wdr[RTQ_WR_INDEX(rg, kc, Kc, li, j)] = d;
    }
  }
}

// GGUF Q4_K / Q6_K super-blocks (ggml layouts) -> the Q4_0 / Q8_0 code layouts, the integer
// sub-block scales (wd) and the fp16 super-block scales (wsb), see rtq_kargs.h.
//   Q4_K (144 B): fp16 d, fp16 dmin, 12 bytes of 6-bit (sc, m) for 8 sub-blocks, 128 bytes of
//     nibbles: sub-block 2c takes the low nibbles of bytes 32c..32c+31, sub-block 2c+1 the high;
//     sub-block j < 4: sc = s[j] & 63, m = s[j+4] & 63; j >= 4: the low / high nibble of s[j+4]
//     with the top two bits of s[j-4] (sc) / s[j] (m) above them.
//   Q6_K (210 B): ql[128], qh[64], int8 sc[16], fp16 d; element 128h + 32m + l has the low four
//     bits of ql[64h + l + 32(m & 1)] (low nibble for m < 2, else high) and the two bits
//     (qh[32h + l] >> 2m) & 3 above them, minus 32; sc[e / 16] scales element e.
void repack_kquant(int type, const uint8_t* src, int64_t N, int64_t K, int64_t Np, int64_t Kp, uint8_t* wq,
                   uint16_t* wd, uint32_t* wsb) {
  const int64_t Kc = Kp / 128, Ksb = Kp / 256, nsb = K / 256, bb = block_bytes(type), rb = nsb * bb;
  const bool q4k = type == RTQ_TYPE_Q4_K;
  for (int64_t n = 0; n < Np; n++) {
    const int64_t rg = n / 16, li = n % 16;
    for (int64_t sb = 0; sb < Ksb; sb++) {
      const uint8_t* blk = (n < N && sb < nsb) ? src + n * rb + sb * bb : nullptr;
      uint32_t dd = 0;
      if (blk) dd = q4k ? (uint32_t)le16(blk) | ((uint32_t)le16(blk + 2) << 16) : (uint32_t)le16(blk + 208);
      wsb[RTQ_WSB_INDEX(rg, sb, Ksb, li)] = dd;
      for (int jj = 0; jj < 8; jj++) {
        const int64_t b = sb * 8 + jj, kc = b / 4, j = b % 4;
        uint8_t codes[32] = {};
        uint16_t word = 0;
        if (blk && q4k) {
          const uint8_t* sc = blk + 4;
          const int s6 = jj < 4 ? sc[jj] & 63 : (sc[jj + 4] & 0xF) | ((sc[jj - 4] >> 6) << 4);
          const int m6 = jj < 4 ? sc[jj + 4] & 63 : (sc[jj + 4] >> 4) | ((sc[jj] >> 6) << 4);
          word = (uint16_t)(s6 | (m6 << 8));
          const uint8_t* qs = blk + 16 + 32 * (jj / 2);
          const int sh = (jj & 1) ? 4 : 0;
          for (int e = 0; e < 16; e++)
            codes[e] = (uint8_t)(((qs[e] >> sh) & 0xF) | (((qs[e + 16] >> sh) & 0xF) << 4));
        } else if (blk) {
          const int h = jj / 4, m = jj % 4;
          const uint8_t* ql = blk + 64 * h + 32 * (m & 1);
          const uint8_t* qh = blk + 128 + 32 * h;
          for (int l = 0; l < 32; l++) {
            const int lo = (m < 2) ? (ql[l] & 0xF) : (ql[l] >> 4);
            const int hi = (qh[l] >> (2 * m)) & 3;
            codes[l] = (uint8_t)(int8_t)((lo | (hi << 4)) - 32);
          }
          word = (uint16_t)(blk[192 + 2 * jj] | (blk[193 + 2 * jj] << 8));
        }
        place_codes(!q4k, codes, rg, kc, li, j, Kc, wq);
        wd[RTQ_WR_INDEX(rg, kc, Kc, li, j)] = word;
      }
    }
  }
}

}  // namespace

rtq_status rtq_model_launch(rtq_ctx* c, int km, dim3 grid, dim3 block, hipStream_t s, const void* args) {
  if (km < 0 || km >= KM_COUNT) return fail(RTQ_ERR_INVALID, "bad decoder kernel id %d", km);
  return launch_raw(c, K_MODEL + km, grid, block, s, const_cast<void*>(args), 0);
}

int rtq_ctx_device_id(const rtq_ctx* c) { return c ? c->device : -1; }
int rtq_ctx_cu_count(const rtq_ctx* c) { return c ? (int)c->cu_count : 256; }
uint64_t rtq_ctx_ws_gen(const rtq_ctx* c) { return c ? c->ws_gen : 0; }
bool rtq_ctx_timing_on(const rtq_ctx* c) { return c && c->timing; }

// error reporting shared with the other translation units of the library (rtq_gguf.cpp, rtq_model.cpp)
rtq_status rtq_fail(rtq_status st, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return st;
}

// ====================================================================== C ABI
extern "C" {

const char* rtq_version(void) { return "rtq 0.1 gfx950"; }
const char* rtq_last_error(void) { return g_err.c_str(); }

rtq_status rtq_ctx_create(int device, rtq_ctx** out) {
  if (!out) return fail(RTQ_ERR_INVALID, "null out");
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return fail(RTQ_ERR_NO_DEVICE, "no HIP device visible");
  if (device < 0 || device >= n) return fail(RTQ_ERR_INVALID, "device %d out of range (%d devices)", device, n);
  HIP_TRY(hipSetDevice(device));
  hipDeviceProp_t prop;
  HIP_TRY(hipGetDeviceProperties(&prop, device));
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(RTQ_ERR_NO_DEVICE, "device %d is %s; this library is built for gfx950 only", device, prop.gcnArchName);
  rtq_ctx* c = new rtq_ctx();
  c->device = device;
  c->cu_count = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
  if (const char* e = getenv("RTQ_DX_SPLITS")) c->dx_splits = atoi(e);
  if (const char* e = getenv("RTQ_DX_WPC")) c->dx_wpc = std::min(std::max(atoi(e), 1), 4);
  if (const char* e = getenv("RTQ_GTOK")) c->gtok = atoi(e);
  if (const char* e = getenv("RTQ_DX_WIDE")) c->dx_wide = atoi(e) ? 1 : 0;
  if (const char* e = getenv("RTQ_DX_32")) c->dx_32 = std::min(std::max(atoi(e), 0), 2);
  if (const char* e = getenv("RTQ_FWD_WAVES")) c->fwd_waves = atoi(e) == 4 ? 4 : 8;
  if (const char* e = getenv("RTQ_FWD_MM")) c->fwd_mm = std::min(std::max(atoi(e), 0), 3);
  if (const char* e = getenv("RTQ_FWD_I8")) c->fwd_i8 = std::min(std::max(atoi(e), -1), 1);
  if (const char* e = getenv("RTQ_FWD_MMK")) c->fwd_mmk = std::min(std::max(atoi(e), -1), 2);
  if (const char* e = getenv("RTQ_GEMVQ")) c->gemvq = atoi(e) ? 1 : 0;
  if (const char* e = getenv("RTQ_DXV")) c->dxv = atoi(e) ? 1 : 0;
  if (const char* e = getenv("RTQ_DXV_WPC")) c->dxv_wpc = std::max(1, std::min(16, atoi(e)));
  if (const char* e = getenv("RTQ_GEMVQ_WPC")) c->gemvq_wpc = std::min(std::max(atoi(e), 0), 32);
  if (const char* e = getenv("RTQ_FWD_RG")) c->fwd_rg = std::min(std::max(atoi(e), 1), 3);
  if (const char* e = getenv("RTQ_ACT_TT")) c->act_tt = atoi(e) <= 4 ? 4 : atoi(e) <= 8 ? 8 : 16;
  if (const char* e = getenv("RTQ_G64_MIN")) c->g64_min = atoi(e);
  hipError_t e = hipModuleLoadData(&c->mod, rtq_hsaco_begin);
  if (e != hipSuccess) {
    delete c;
    return fail(RTQ_ERR_NO_DEVICE, "hipModuleLoadData: %s", hipGetErrorString(e));
  }
  for (int k = 0; k < K_COUNT; k++) {
    e = hipModuleGetFunction(&c->fn[k], c->mod, kKernelNames[k]);
    if (e != hipSuccess) {
      (void)hipModuleUnload(c->mod);
      delete c;
      return fail(RTQ_ERR_NO_DEVICE, "kernel %s missing from code object: %s", kKernelNames[k], hipGetErrorString(e));
    }
  }
  if (const rtq_status st = rtq_scratch_setup(device); st != RTQ_OK) {  // rtq_linear_forward_noalloc_d's array
    (void)hipModuleUnload(c->mod);
    delete c;
    return st;
  }
  e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);  // default priority
  if (e != hipSuccess) {
    rtq_ctx_destroy(c);
    return fail(RTQ_ERR_HIP, "hipStreamCreate: %s", hipGetErrorString(e));
  }
  *out = c;
  return RTQ_OK;
}

void rtq_ctx_destroy(rtq_ctx* c) {
  if (!c) return;
  (void)hipSetDevice(c->device);
  (void)hipDeviceSynchronize();
  for (auto& p : c->pending) {
    (void)hipEventDestroy(p.a);
    (void)hipEventDestroy(p.b);
  }
  for (auto e : c->free_events) (void)hipEventDestroy(e);
  if (c->ws) (void)hipFree(c->ws);
  if (c->stream) (void)hipStreamDestroy(c->stream);
  if (c->mod) (void)hipModuleUnload(c->mod);
  delete c;
}

void* rtq_ctx_stream(rtq_ctx* c) { return c ? (void*)c->stream : nullptr; }

rtq_status rtq_ctx_reserve(rtq_ctx* c, int64_t max_t, int64_t max_rows, int64_t max_cols, int64_t max_rank) {
  if (!c) return fail(RTQ_ERR_INVALID, "null context");
  std::lock_guard<std::mutex> lk(c->mu);
  HIP_TRY(hipSetDevice(c->device));
  rtq_weight fake;
  fake.rows = max_rows;
  fake.cols = max_cols;
  fake.Np = roundup(max_rows, RTQ_ROW_PAD);
  fake.Kp = roundup(max_cols, RTQ_CHUNK_Q);
  fake.type = RTQ_TYPE_Q4_0;
  size_t need = fwd_ws_bytes(fwd_plan(&fake, max_t, max_rank));
  for (int64_t t : {std::min<int64_t>(max_t, 16), max_t})  // both dx paths
    need = std::max(need, bwd_ws_bytes(c, &fake, t, max_rank));
  RTQ_TRY(ensure_ws(c, need));
  return RTQ_OK;
}

rtq_status rtq_ctx_set_timing(rtq_ctx* c, int enable, const char* only_kernel) {
  if (!c) return fail(RTQ_ERR_INVALID, "null context");
  std::lock_guard<std::mutex> lk(c->mu);
  int only = -1;
  if (only_kernel) {
    for (int k = 0; k < K_COUNT; k++)
      if (strcmp(only_kernel, kKernelNames[k]) == 0) only = k;
    if (only < 0) return fail(RTQ_ERR_INVALID, "unknown kernel %s", only_kernel);
  }
  c->timing = enable != 0;
  c->timing_only = only;
  return RTQ_OK;
}

static void fold_timing(rtq_ctx* c) {
  if (c->pending.empty()) return;
  (void)hipSetDevice(c->device);
  (void)hipDeviceSynchronize();
  for (auto& p : c->pending) {
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, p.a, p.b) == hipSuccess) {
      c->t_launches[p.kid] += 1;
      c->t_ms[p.kid] += ms;
      c->t_flops[p.kid] += p.flops;
      c->t_bytes[p.kid] += p.bytes;
    }
    c->free_events.push_back(p.a);
    c->free_events.push_back(p.b);
  }
  c->pending.clear();
}

int rtq_ctx_timing_count(rtq_ctx* c) {
  if (!c) return 0;
  std::lock_guard<std::mutex> lk(c->mu);
  fold_timing(c);
  return K_COUNT;
}

rtq_status rtq_ctx_timing_get(rtq_ctx* c, int i, const char** name, int64_t* launches, double* total_ms) {
  if (!c || i < 0 || i >= K_COUNT) return fail(RTQ_ERR_INVALID, "bad timing index");
  std::lock_guard<std::mutex> lk(c->mu);
  fold_timing(c);
  if (name) *name = kKernelNames[i];
  if (launches) *launches = c->t_launches[i];
  if (total_ms) *total_ms = c->t_ms[i];
  return RTQ_OK;
}

rtq_status rtq_ctx_timing_work(rtq_ctx* c, int i, double* flops, double* bytes) {
  if (!c || i < 0 || i >= K_COUNT) return fail(RTQ_ERR_INVALID, "bad timing index");
  std::lock_guard<std::mutex> lk(c->mu);
  fold_timing(c);
  if (flops) *flops = c->t_flops[i];
  if (bytes) *bytes = c->t_bytes[i];
  return RTQ_OK;
}

void rtq_ctx_timing_reset(rtq_ctx* c) {
  if (!c) return;
  std::lock_guard<std::mutex> lk(c->mu);
  fold_timing(c);
  for (int k = 0; k < K_COUNT; k++) {
    c->t_launches[k] = 0;
    c->t_ms[k] = 0.0;
    c->t_flops[k] = c->t_bytes[k] = 0.0;
  }
}

rtq_status rtq_weight_create(rtq_ctx* c, int type, const void* blocks, size_t nbytes, int64_t rows, int64_t cols,
                             rtq_weight** out) {
  if (!c || !out) return fail(RTQ_ERR_INVALID, "null context/out");
  *out = nullptr;
  if (!supported(type)) return fail(RTQ_ERR_UNSUPPORTED, "ggml type %d is not supported", type);
  if (rows <= 0 || cols <= 0) return fail(RTQ_ERR_INVALID, "empty weight %lldx%lld", (long long)rows, (long long)cols);
  if (cols % block_elems(type))
    return fail(RTQ_ERR_INVALID, "cols %lld not a multiple of the block size %lld", (long long)cols,
                (long long)block_elems(type));
  if (rows > (1LL << 30) || cols > (1LL << 24)) return fail(RTQ_ERR_INVALID, "weight too large");
  const size_t expect = (size_t)rows * (size_t)(cols / block_elems(type) * block_bytes(type));
  if (!blocks || nbytes != expect)
    return fail(RTQ_ERR_INVALID, "weight bytes %zu != rows*row_bytes %zu", nbytes, expect);
  std::lock_guard<std::mutex> lk(c->mu);
  HIP_TRY(hipSetDevice(c->device));
  rtq_weight* w = new rtq_weight();
  w->ctx = c;
  w->type = type;
  w->rows = rows;
  w->cols = cols;
  w->Np = roundup(rows, RTQ_ROW_PAD);
  w->Kp = roundup(cols, RTQ_CHUNK_Q);
  w->gguf_bytes = expect;
  if (is_dense(type)) {  // trainer-native storage, uploaded as it is
    if ((uint64_t)rows * (uint64_t)cols * 4u >= (1ull << 31) * 2u) {
      delete w;
      return fail(RTQ_ERR_INVALID, "weight %lldx%lld too large for the f32 GEMM path", (long long)rows, (long long)cols);
    }
    hipError_t e = hipMalloc(&w->dmem, expect);
    if (e != hipSuccess) {
      delete w;
      return fail(RTQ_ERR_HIP, "hipMalloc(%zu): %s", expect, hipGetErrorString(e));
    }
    e = hipMemcpy(w->dmem, blocks, expect, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
      (void)hipFree(w->dmem);
      delete w;
      return fail(RTQ_ERR_HIP, "upload: %s", hipGetErrorString(e));
    }
    if (type == RTQ_TYPE_TQ8_0) {
      w->wsc = reinterpret_cast<const float*>(w->dmem);
      w->wq = (char*)w->dmem + (size_t)rows * (cols / 32) * 4;
    } else {
      w->wq = w->dmem;
    }
    *out = w;
    return RTQ_OK;
  }
  const int64_t nbp = w->Kp / 32;
  const size_t q_bytes = (size_t)w->Np * nbp * (byte_codes(type) ? 32 : 16);
  const size_t d_bytes = (size_t)w->Np * nbp * 2;
  const size_t e_bytes = is_kquant(type) ? (size_t)w->Np * (w->Kp / 256) * 4 : 0;
  const size_t r_bytes = is_kquant(type) ? 0 : d_bytes;  // row-major copy of the fp16 scales
  const size_t q_off = 0, d_off = roundup((int64_t)q_bytes, 256), e_off = d_off + roundup((int64_t)d_bytes, 256);
  const size_t r_off = e_off + roundup((int64_t)e_bytes, 256);
  const size_t total = r_off + roundup((int64_t)r_bytes, 256);
  if (q_bytes >= (1ull << 31)) {  // the kernels address codes with 32-bit buffer offsets
    delete w;
    return fail(RTQ_ERR_INVALID, "weight %lldx%lld: %zu code bytes exceed 2 GiB", (long long)rows, (long long)cols, q_bytes);
  }
  std::vector<uint8_t> host(total, 0);
  if (is_kquant(type))
    repack_kquant(type, (const uint8_t*)blocks, rows, cols, w->Np, w->Kp, host.data() + q_off,
                  reinterpret_cast<uint16_t*>(host.data() + d_off), reinterpret_cast<uint32_t*>(host.data() + e_off));
  else
    repack_q32(type, (const uint8_t*)blocks, rows, cols, w->Np, w->Kp, host.data() + q_off,
               reinterpret_cast<uint16_t*>(host.data() + d_off), reinterpret_cast<uint16_t*>(host.data() + r_off));
  {  // bound of |dequantised value| -> sigma
    double bound = 0.0;
    if (is_kquant(type)) {
      const uint32_t* sb = reinterpret_cast<const uint32_t*>(host.data() + e_off);
      for (size_t i = 0; i < e_bytes / 4; i++) {
        const double d = fabs((double)f16_bits_to_f32((uint16_t)(sb[i] & 0xffffu)));
        const double dm = fabs((double)f16_bits_to_f32((uint16_t)(sb[i] >> 16)));
        bound = std::max(bound, type == RTQ_TYPE_Q4_K ? d * 63.0 * 15.0 + dm * 63.0 : d * 128.0 * 32.0);
      }
    } else {
      const uint16_t* dd = reinterpret_cast<const uint16_t*>(host.data() + d_off);
      for (size_t i = 0; i < d_bytes / 2; i++)
        bound = std::max(bound, fabs((double)f16_bits_to_f32(dd[i])) * (type == RTQ_TYPE_Q4_0 ? 8.0 : 128.0));
    }
    int sigma = 0;
    while (sigma < 60 && bound * std::ldexp(1.0, -sigma) >= 32768.0) sigma++;
    w->dx_wsc = std::ldexp(1.0f, -sigma);
    w->dx_wunsc = std::ldexp(1.0f, sigma);
  }
  hipError_t e = hipMalloc(&w->dmem, total);
  if (e != hipSuccess) {
    delete w;
    return fail(RTQ_ERR_HIP, "hipMalloc(%zu): %s", total, hipGetErrorString(e));
  }
  e = hipMemcpy(w->dmem, host.data(), total, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(w->dmem);
    delete w;
    return fail(RTQ_ERR_HIP, "upload: %s", hipGetErrorString(e));
  }
  w->wq = (char*)w->dmem + q_off;
  w->wd = reinterpret_cast<uint16_t*>((char*)w->dmem + d_off);
  w->wsb = is_kquant(type) ? reinterpret_cast<uint32_t*>((char*)w->dmem + e_off) : nullptr;
  w->wdr = is_kquant(type) ? w->wd : reinterpret_cast<uint16_t*>((char*)w->dmem + r_off);
  *out = w;
  return RTQ_OK;
}

void rtq_weight_destroy(rtq_weight* w) {
  if (!w) return;
  if (w->dmem) {
    std::lock_guard<std::mutex> lk(w->ctx->mu);
    (void)hipSetDevice(w->ctx->device);
    (void)hipDeviceSynchronize();
    (void)hipFree(w->dmem);
  }
  delete w;
}

int64_t rtq_weight_out_dim(const rtq_weight* w) { return w ? w->rows : 0; }
int64_t rtq_weight_in_dim(const rtq_weight* w) { return w ? w->cols : 0; }
size_t rtq_weight_nbytes(const rtq_weight* w) { return w ? w->gguf_bytes : 0; }
int rtq_weight_type(const rtq_weight* w) { return w ? w->type : -1; }

// ------------------------------------------------------------------ device-pointer API
rtq_status rtq_frozen_forward_d(rtq_ctx* c, const rtq_weight* w, const float* x, int64_t t, float* y, void* stream) {
  return rtq_linear_forward_d(c, w, nullptr, nullptr, x, t, y, stream);
}

rtq_status rtq_linear_forward_d(rtq_ctx* c, const rtq_weight* w, const float* bias, const rtq_lora* lora,
                                const float* x, int64_t t, float* y, void* stream) {
  RTQ_TRY(check_weight(c, w));
  RTQ_TRY(check_t(t));
  bool on;
  int64_t r;
  float s;
  RTQ_TRY(check_lora(lora, &on, &r, &s));
  if (t > 0 && (!x || !y)) return fail(RTQ_ERR_INVALID, "null x/y");
  std::lock_guard<std::mutex> lk(c->mu);
  HIP_TRY(hipSetDevice(c->device));
  hipStream_t st = (hipStream_t)stream;  // NULL: the HIP null stream
  FwdPlan p = fwd_plan(w, t, on ? r : 0);
  RTQ_TRY(ensure_ws(c, fwd_ws_bytes(p)));
  Arena ar{(char*)c->ws, c->ws_bytes, 0};
  return enqueue_forward(c, w, x, t, y, bias, on ? lora->a : nullptr, on ? lora->b : nullptr, r, s, nullptr, ar, st);
}

rtq_status rtq_frozen_backward_input_d(rtq_ctx* c, const rtq_weight* w, const float* dy, int64_t t, float* dx,
                                       void* stream) {
  RTQ_TRY(check_weight(c, w));
  RTQ_TRY(check_t(t));
  if (t > 0 && (!dy || !dx)) return fail(RTQ_ERR_INVALID, "null dy/dx");
  std::lock_guard<std::mutex> lk(c->mu);
  HIP_TRY(hipSetDevice(c->device));
  hipStream_t st = (hipStream_t)stream;  // NULL: the HIP null stream
  RTQ_TRY(ensure_ws(c, bwd_ws_bytes(c, w, t, 0)));
  Arena ar{(char*)c->ws, c->ws_bytes, 0};
  return enqueue_backward(c, w, dy, t, dx, true, nullptr, nullptr, nullptr, 0, 0.0f, nullptr, nullptr, ar, st);
}

static rtq_status linear_backward_d(rtq_ctx* c, const rtq_weight* w, const rtq_lora* lora, const float* x,
                                    const float* dy, int64_t t, float* dx, float* ga, float* gb, void* stream,
                                    const RankBlocks* rb, const float* hp_have = nullptr,
                                    const LoraDefer* defer = nullptr) {
  RTQ_TRY(check_weight(c, w));
  RTQ_TRY(check_t(t));
  bool on;
  int64_t r;
  float s;
  RTQ_TRY(check_lora(lora, &on, &r, &s));
  if (t > 0 && (!dy || !dx)) return fail(RTQ_ERR_INVALID, "null dy/dx");
  if (on && t > 0 && (!x || !ga || !gb)) return fail(RTQ_ERR_INVALID, "lora backward needs x, ga and gb");
  std::lock_guard<std::mutex> lk(c->mu);
  HIP_TRY(hipSetDevice(c->device));
  hipStream_t st = (hipStream_t)stream;  // NULL: the HIP null stream
  RTQ_TRY(ensure_ws(c, bwd_ws_bytes(c, w, t, on ? r : 0)));
  Arena ar{(char*)c->ws, c->ws_bytes, 0};
  return enqueue_backward(c, w, dy, t, dx, false, x, on ? lora->a : nullptr, on ? lora->b : nullptr, r, s, ga, gb,
                          ar, st, rb, hp_have, defer);
}

rtq_status rtq_linear_backward_d(rtq_ctx* c, const rtq_weight* w, const rtq_lora* lora, const float* x,
                                 const float* dy, int64_t t, float* dx, float* ga, float* gb, void* stream) {
  return linear_backward_d(c, w, lora, x, dy, t, dx, ga, gb, stream, nullptr);
}

static rtq_status enqueue_rows(rtq_ctx* c, const rtq_weight* w, int64_t r0, int64_t count, float* out,
                               hipStream_t st, const int32_t* idx = nullptr) {
  if (is_dense(w->type)) {  // F32: copy; TQ8_0: 0 + d * q (src/frozen.rs:169-177)
    DenseArgs da{w->type == RTQ_TYPE_F32 ? reinterpret_cast<const float*>(w->wq) : nullptr, w->wsc,
                 reinterpret_cast<const int8_t*>(w->wq), w->rows, w->cols, r0, count, out, nullptr, idx};
    return launch(c, K_DENSE_ROWS, dim3((unsigned)std::min<int64_t>(cdiv(count * w->cols, 256), 8192)), dim3(256), st, da);
  }
  RowArgs ra{w->wq, w->wd, w->wsb, (int)w->Np, (int)w->Kp, (int)w->cols, (int)r0, (int)count, out, idx,
             (int)w->rows};
  const int64_t threads = count * (w->cols / 32);
  return launch(c, K_ROWS + fmt_index(w->type), dim3((unsigned)cdiv(threads, 256)), dim3(256), st, ra);
}

rtq_status rtq_frozen_rows_d(rtq_ctx* c, const rtq_weight* w, int64_t r0, int64_t count, float* out, void* stream) {
  RTQ_TRY(check_weight(c, w));
  if (r0 < 0 || count < 0 || r0 + count > w->rows) return fail(RTQ_ERR_INVALID, "rows out of range");
  if (count == 0) return RTQ_OK;
  if (!out) return fail(RTQ_ERR_INVALID, "null out");
  std::lock_guard<std::mutex> lk(c->mu);
  HIP_TRY(hipSetDevice(c->device));
  return enqueue_rows(c, w, r0, count, out, (hipStream_t)stream);
}

rtq_status rtq_frozen_gather_d(rtq_ctx* c, const rtq_weight* w, const int32_t* ids, int64_t count, float* out,
                               void* stream) {
  RTQ_TRY(check_weight(c, w));
  if (count < 0 || count > (1LL << 24)) return fail(RTQ_ERR_INVALID, "gather count %lld out of range", (long long)count);
  if (count == 0) return RTQ_OK;
  if (!ids || !out) return fail(RTQ_ERR_INVALID, "null ids/out");
  std::lock_guard<std::mutex> lk(c->mu);
  HIP_TRY(hipSetDevice(c->device));
  return enqueue_rows(c, w, 0, count, out, (hipStream_t)stream, ids);
}

// ------------------------------------------------------------------ LM head + cross-entropy
namespace {

struct HeadPlan {
  int G, L;
  size_t bytes;  // workspace: head buffers + the larger of the lm_head forward / backward workspaces
};

HeadPlan head_plan(const rtq_ctx* c, const rtq_weight* w, int64_t n, bool grad) {
  const int64_t V = w->rows, d = w->cols;
  // enough (slice, row) workgroups to fill the chip four times, slices of at least 4096 logits
  int64_t G = std::min<int64_t>(std::max<int64_t>(cdiv(4 * c->cu_count, n), 1), std::max<int64_t>(V / 4096, 1));
  G = std::min<int64_t>(G, 64);
  const int64_t L = roundup(cdiv(V, G), 4);
  G = cdiv(V, L);
  size_t b = (size_t)(n * d) * 4 * 2 + (size_t)n * 4 + (size_t)(n * V) * 4 + (size_t)(n * G) * 12 + 8 * 256;
  size_t sub = fwd_ws_bytes(fwd_plan(w, n, 0));
  if (grad) sub = std::max(sub, bwd_ws_bytes(c, w, n, 0));
  return HeadPlan{(int)G, (int)L, b + sub};
}

rtq_status enqueue_head(rtq_ctx* c, const rtq_weight* w, const float* norm, float eps, float off, const float* x,
                        int64_t t, const int32_t* pos, const int32_t* tok, const float* wts, int64_t n, float* logp,
                        int32_t* hit, float* dx, const HeadPlan& hp, Arena& ar, hipStream_t st) {
  const int64_t V = w->rows, d = w->cols;
  float* ns = ar.take<float>((size_t)(n * d));
  float* inv = ar.take<float>((size_t)n);
  float* logits = ar.take<float>((size_t)(n * V));
  float* pmax = ar.take<float>((size_t)(n * hp.G));
  double* psum = ar.take<double>((size_t)(n * hp.G));
  float* dns = wts ? ar.take<float>((size_t)(n * d)) : nullptr;
  if (ar.off > ar.cap) return fail(RTQ_ERR_INVALID, "internal: workspace too small");
  HeadArgs ha{x,   pos,   tok,    wts,  norm,      eps,  off,    (int)t, (int)d, (int)n, (int)V, hp.G, hp.L,
              ns,  inv,   logits, pmax, psum,      logp, hit,    dns,    dx};
  RTQ_TRY(launch(c, K_HEAD_NORM, dim3((unsigned)n), dim3(256), st, ha));
  Arena fa = ar;
  RTQ_TRY(enqueue_forward(c, w, ns, n, logits, nullptr, nullptr, nullptr, 0, 0.0f, nullptr, fa, st));
  const dim3 sg((unsigned)hp.G, (unsigned)n);
  RTQ_TRY(launch(c, K_HEAD_MAX, sg, dim3(256), st, ha));
  RTQ_TRY(launch(c, K_HEAD_SUM, sg, dim3(256), st, ha));
  RTQ_TRY(launch(c, K_HEAD_GRAD, sg, dim3(256), st, ha));
  if (!wts) return RTQ_OK;
  Arena ba = ar;
  RTQ_TRY(enqueue_backward(c, w, logits, n, dns, false, nullptr, nullptr, nullptr, 0, 0.0f, nullptr, nullptr, ba, st));
  FillArgs fz{dx, t * d};
  RTQ_TRY(launch(c, K_FILL, dim3((unsigned)std::min<int64_t>(cdiv(t * d, 256), 4096)), dim3(256), st, fz));
  return launch(c, K_HEAD_NORM_BWD, dim3((unsigned)n), dim3(256), st, ha);
}

rtq_status check_head(rtq_ctx* c, const rtq_weight* w, const float* norm, const float* x, int64_t t, const int32_t* pos,
                      const int32_t* tok, const float* wts, int64_t n, const float* logp, const float* dx) {
  RTQ_TRY(check_weight(c, w));
  RTQ_TRY(check_t(t));
  if (n < 0 || n > 65535) return fail(RTQ_ERR_INVALID, "target count %lld out of range [0, 65535]", (long long)n);
  if (n > 0 && (!norm || !x || !pos || !tok || !logp)) return fail(RTQ_ERR_INVALID, "null norm/x/pos/tok/logp");
  if (n > 0 && wts && !dx) return fail(RTQ_ERR_INVALID, "weights given without dx");
  if ((double)n * (double)w->rows > 4e9) return fail(RTQ_ERR_INVALID, "n x vocab logits too large");
  return RTQ_OK;
}

}  // namespace

rtq_status rtq_lm_head_d(rtq_ctx* c, const rtq_weight* w, const float* norm, float eps, float offset, const float* x,
                         int64_t t, const int32_t* pos, const int32_t* tok, const float* weights, int64_t n,
                         float* logp, int32_t* hit, float* dx, void* stream) {
  RTQ_TRY(check_head(c, w, norm, x, t, pos, tok, weights, n, logp, dx));
  if (n > 0 && !hit) return fail(RTQ_ERR_INVALID, "null hit");
  std::lock_guard<std::mutex> lk(c->mu);
  HIP_TRY(hipSetDevice(c->device));
  hipStream_t st = (hipStream_t)stream;
  if (n == 0) {
    if (weights && dx && t > 0) {
      FillArgs fz{dx, t * w->cols};
      return launch(c, K_FILL, dim3((unsigned)std::min<int64_t>(cdiv(t * w->cols, 256), 4096)), dim3(256), st, fz);
    }
    return RTQ_OK;
  }
  const HeadPlan hp = head_plan(c, w, n, weights != nullptr);
  RTQ_TRY(ensure_ws(c, hp.bytes));
  Arena ar{(char*)c->ws, c->ws_bytes, 0};
  return enqueue_head(c, w, norm, eps, offset, x, t, pos, tok, weights, n, logp, hit, dx, hp, ar, st);
}

// ------------------------------------------------------------------ host-pointer API
namespace {

struct HostCall {
  rtq_ctx* c;
  std::unique_lock<std::mutex> lk;
  explicit HostCall(rtq_ctx* ctx) : c(ctx), lk(ctx->mu) {}
};

static rtq_status h2d(void* d, const void* h, size_t bytes, hipStream_t st) {
  if (bytes) HIP_TRY(hipMemcpyAsync(d, h, bytes, hipMemcpyHostToDevice, st));
  return RTQ_OK;
}
static rtq_status d2h(void* h, const void* d, size_t bytes, hipStream_t st) {
  if (bytes) HIP_TRY(hipMemcpyAsync(h, d, bytes, hipMemcpyDeviceToHost, st));
  return RTQ_OK;
}

}  // namespace

rtq_status rtq_linear_forward(rtq_ctx* c, const rtq_weight* w, const float* bias, const rtq_lora* lora, const float* x,
                              int64_t t, float* y) {
  RTQ_TRY(check_weight(c, w));
  RTQ_TRY(check_t(t));
  bool on;
  int64_t r;
  float s;
  RTQ_TRY(check_lora(lora, &on, &r, &s));
  if (t == 0) return RTQ_OK;
  if (!x || !y) return fail(RTQ_ERR_INVALID, "null x/y");
  HostCall hc(c);
  HIP_TRY(hipSetDevice(c->device));
  hipStream_t st = c->stream;
  const int64_t N = w->rows, K = w->cols;
  FwdPlan p = fwd_plan(w, t, on ? r : 0);
  const size_t io = (size_t)(t * K + t * N + (bias ? N : 0) + (on ? r * K + N * r : 0)) * 4 + 6 * 256;
  RTQ_TRY(ensure_ws(c, fwd_ws_bytes(p) + io));
  Arena ar{(char*)c->ws, c->ws_bytes, 0};
  float* xd = ar.take<float>((size_t)(t * K));
  float* yd = ar.take<float>((size_t)(t * N));
  float* bd = bias ? ar.take<float>((size_t)N) : nullptr;
  float* ad = on ? ar.take<float>((size_t)(r * K)) : nullptr;
  float* bld = on ? ar.take<float>((size_t)(N * r)) : nullptr;
  RTQ_TRY(h2d(xd, x, (size_t)(t * K) * 4, st));
  if (bd) RTQ_TRY(h2d(bd, bias, (size_t)N * 4, st));
  if (on) {
    RTQ_TRY(h2d(ad, lora->a, (size_t)(r * K) * 4, st));
    RTQ_TRY(h2d(bld, lora->b, (size_t)(N * r) * 4, st));
  }
  RTQ_TRY(enqueue_forward(c, w, xd, t, yd, bd, ad, bld, on ? r : 0, s, nullptr, ar, st));
  RTQ_TRY(d2h(y, yd, (size_t)(t * N) * 4, st));
  HIP_TRY(hipStreamSynchronize(st));
  return RTQ_OK;
}

rtq_status rtq_frozen_forward(rtq_ctx* c, const rtq_weight* w, const float* x, int64_t t, float* y) {
  return rtq_linear_forward(c, w, nullptr, nullptr, x, t, y);
}

static rtq_status backward_host(rtq_ctx* c, const rtq_weight* w, const rtq_lora* lora, const float* x, const float* dy,
                                int64_t t, float* dx, float* ga, float* gb, bool linear) {
  RTQ_TRY(check_weight(c, w));
  RTQ_TRY(check_t(t));
  bool on;
  int64_t r;
  float s;
  RTQ_TRY(check_lora(linear ? lora : nullptr, &on, &r, &s));
  if (t == 0) return RTQ_OK;
  if (!dy || !dx) return fail(RTQ_ERR_INVALID, "null dy/dx");
  if (on && (!x || !ga || !gb)) return fail(RTQ_ERR_INVALID, "lora backward needs x, ga and gb");
  HostCall hc(c);
  HIP_TRY(hipSetDevice(c->device));
  hipStream_t st = c->stream;
  const int64_t N = w->rows, K = w->cols;
  const size_t io = (size_t)(t * N + t * K + (on ? t * K + 2 * r * K + 2 * N * r : 0)) * 4 + 8 * 256;
  RTQ_TRY(ensure_ws(c, bwd_ws_bytes(c, w, t, on ? r : 0) + io));
  Arena ar{(char*)c->ws, c->ws_bytes, 0};
  float* dyd = ar.take<float>((size_t)(t * N));
  float* dxd = ar.take<float>((size_t)(t * K));
  float *xd = nullptr, *ad = nullptr, *bld = nullptr, *gad = nullptr, *gbd = nullptr;
  if (on) {
    xd = ar.take<float>((size_t)(t * K));
    ad = ar.take<float>((size_t)(r * K));
    bld = ar.take<float>((size_t)(N * r));
    gad = ar.take<float>((size_t)(r * K));
    gbd = ar.take<float>((size_t)(N * r));
  }
  RTQ_TRY(h2d(dyd, dy, (size_t)(t * N) * 4, st));
  if (!linear) RTQ_TRY(h2d(dxd, dx, (size_t)(t * K) * 4, st));  // FrozenMatmul accumulates into dx
  if (on) {
    RTQ_TRY(h2d(xd, x, (size_t)(t * K) * 4, st));
    RTQ_TRY(h2d(ad, lora->a, (size_t)(r * K) * 4, st));
    RTQ_TRY(h2d(bld, lora->b, (size_t)(N * r) * 4, st));
    RTQ_TRY(h2d(gad, ga, (size_t)(r * K) * 4, st));
    RTQ_TRY(h2d(gbd, gb, (size_t)(N * r) * 4, st));
  }
  RTQ_TRY(enqueue_backward(c, w, dyd, t, dxd, !linear, xd, ad, bld, on ? r : 0, s, gad, gbd, ar, st));
  RTQ_TRY(d2h(dx, dxd, (size_t)(t * K) * 4, st));
  if (on) {
    RTQ_TRY(d2h(ga, gad, (size_t)(r * K) * 4, st));
    RTQ_TRY(d2h(gb, gbd, (size_t)(N * r) * 4, st));
  }
  HIP_TRY(hipStreamSynchronize(st));
  return RTQ_OK;
}

rtq_status rtq_frozen_backward_input(rtq_ctx* c, const rtq_weight* w, const float* dy, int64_t t, float* dx) {
  return backward_host(c, w, nullptr, nullptr, dy, t, dx, nullptr, nullptr, false);
}

rtq_status rtq_linear_backward(rtq_ctx* c, const rtq_weight* w, const rtq_lora* lora, const float* x, const float* dy,
                               int64_t t, float* dx, float* ga, float* gb) {
  return backward_host(c, w, lora, x, dy, t, dx, ga, gb, true);
}

rtq_status rtq_frozen_row(rtq_ctx* c, const rtq_weight* w, int64_t r, float* out) {
  RTQ_TRY(check_weight(c, w));
  if (r < 0 || r >= w->rows) return fail(RTQ_ERR_INVALID, "row %lld out of range", (long long)r);
  if (!out) return fail(RTQ_ERR_INVALID, "null out");
  HostCall hc(c);
  HIP_TRY(hipSetDevice(c->device));
  RTQ_TRY(ensure_ws(c, (size_t)w->cols * 4 + 256));
  float* od = (float*)c->ws;
  RTQ_TRY(enqueue_rows(c, w, r, 1, od, c->stream));
  RTQ_TRY(d2h(out, od, (size_t)w->cols * 4, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  return RTQ_OK;
}

/* embed_tokens (src/model.rs:446-454): out[i] = row(ids[i]) */
rtq_status rtq_frozen_gather(rtq_ctx* c, const rtq_weight* w, const int32_t* ids, int64_t count, float* out) {
  RTQ_TRY(check_weight(c, w));
  if (count < 0 || count > (1LL << 24)) return fail(RTQ_ERR_INVALID, "gather count %lld out of range", (long long)count);
  if (count == 0) return RTQ_OK;
  if (!ids || !out) return fail(RTQ_ERR_INVALID, "null ids/out");
  for (int64_t i = 0; i < count; i++)
    if (ids[i] < 0 || ids[i] >= w->rows)
      return fail(RTQ_ERR_INVALID, "token %d out of vocab (%lld rows)", ids[i], (long long)w->rows);
  HostCall hc(c);
  HIP_TRY(hipSetDevice(c->device));
  const size_t ob = (size_t)(count * w->cols) * 4;
  RTQ_TRY(ensure_ws(c, ob + (size_t)count * 4 + 512));
  Arena ar{(char*)c->ws, c->ws_bytes, 0};
  float* od = ar.take<float>((size_t)(count * w->cols));
  int32_t* idd = ar.take<int32_t>((size_t)count);
  RTQ_TRY(h2d(idd, ids, (size_t)count * 4, c->stream));
  RTQ_TRY(enqueue_rows(c, w, 0, count, od, c->stream, idd));
  RTQ_TRY(d2h(out, od, ob, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  return RTQ_OK;
}

/* Model::head (src/model.rs:561-609) with host arrays; targets out of range are rejected (the
 * reference asserts, :575) */
rtq_status rtq_lm_head(rtq_ctx* c, const rtq_weight* w, const float* norm, float eps, float offset, const float* x,
                       int64_t t, const int32_t* pos, const int32_t* tok, const float* weights, int64_t n, float* logp,
                       int64_t* hits, float* dx) {
  RTQ_TRY(check_head(c, w, norm, x, t, pos, tok, weights, n, logp, dx));
  for (int64_t i = 0; i < n; i++)
    if (pos[i] < 0 || pos[i] >= t || tok[i] < 0 || tok[i] >= w->rows)
      return fail(RTQ_ERR_INVALID, "target %lld (pos %d, token %d) out of range", (long long)i, pos[i], tok[i]);
  const int64_t d = w->cols;
  if (hits) *hits = 0;
  if (n == 0) {
    if (weights && dx) memset(dx, 0, (size_t)(t * d) * 4);
    return RTQ_OK;
  }
  HostCall hc(c);
  HIP_TRY(hipSetDevice(c->device));
  hipStream_t st = c->stream;
  const HeadPlan hp = head_plan(c, w, n, weights != nullptr);
  const size_t io = (size_t)(t * d + d + n * 5 + (weights ? t * d : 0)) * 4 + 8 * 256;
  RTQ_TRY(ensure_ws(c, hp.bytes + io));
  Arena ar{(char*)c->ws, c->ws_bytes, 0};
  float* xd = ar.take<float>((size_t)(t * d));
  float* nd = ar.take<float>((size_t)d);
  int32_t* pd = ar.take<int32_t>((size_t)n);
  int32_t* kd = ar.take<int32_t>((size_t)n);
  float* wd = weights ? ar.take<float>((size_t)n) : nullptr;
  float* ld = ar.take<float>((size_t)n);
  int32_t* hd = ar.take<int32_t>((size_t)n);
  float* dxd = weights ? ar.take<float>((size_t)(t * d)) : nullptr;
  RTQ_TRY(h2d(xd, x, (size_t)(t * d) * 4, st));
  RTQ_TRY(h2d(nd, norm, (size_t)d * 4, st));
  RTQ_TRY(h2d(pd, pos, (size_t)n * 4, st));
  RTQ_TRY(h2d(kd, tok, (size_t)n * 4, st));
  if (wd) RTQ_TRY(h2d(wd, weights, (size_t)n * 4, st));
  RTQ_TRY(enqueue_head(c, w, nd, eps, offset, xd, t, pd, kd, wd, n, ld, hd, dxd, hp, ar, st));
  std::vector<int32_t> hv((size_t)n);
  RTQ_TRY(d2h(logp, ld, (size_t)n * 4, st));
  RTQ_TRY(d2h(hv.data(), hd, (size_t)n * 4, st));
  if (dxd) RTQ_TRY(d2h(dx, dxd, (size_t)(t * d) * 4, st));
  HIP_TRY(hipStreamSynchronize(st));
  if (hits) {
    int64_t s = 0;
    for (int32_t h : hv) s += h;
    *hits = s;
  }
  return RTQ_OK;
}

// ------------------------------------------------------------------ parity / debug
int64_t rtq_debug_isums_per_row(const rtq_weight* w) {
  if (!w || is_dense(w->type)) return 0;
  if (is_q32(w->type)) return w->cols / 32;
  if (w->type == RTQ_TYPE_Q4_K) return 2 * (w->cols / 256);
  return w->cols / 256;
}

rtq_status rtq_debug_quantize_acts(rtq_ctx* c, const rtq_weight* w, const float* x, int64_t t, void* out) {
  RTQ_TRY(check_weight(c, w));
  RTQ_TRY(check_t(t));
  if (is_dense(w->type)) return fail(RTQ_ERR_UNSUPPORTED, "trainer-native weights take f32 activations");
  if (t == 0) return RTQ_OK;
  if (!x || !out) return fail(RTQ_ERR_INVALID, "null x/out");
  HostCall hc(c);
  HIP_TRY(hipSetDevice(c->device));
  hipStream_t st = c->stream;
  const int64_t K = w->cols;
  FwdPlan p = fwd_plan(w, t, 0);
  RTQ_TRY(ensure_ws(c, fwd_ws_bytes(p) + (size_t)(t * K) * 4 + 256));
  Arena ar{(char*)c->ws, c->ws_bytes, 0};
  float* xdv = ar.take<float>((size_t)(t * K));
  void* xq = ar.take<char>(p.xq_bytes);
  float* xs = ar.take<float>(p.xd_floats);
  RTQ_TRY(h2d(xdv, x, (size_t)(t * K) * 4, st));
  const bool kq = is_kquant(w->type);
  ActArgs aa{xdv, (int)t, (int)K, (int)p.Tp, (int)w->Kp, xq, xs, nullptr, 0.0f, nullptr, 0, nullptr, nullptr, 0, nullptr};
  RTQ_TRY(launch(c, kq ? K_ACT_PREP_K : K_ACT_PREP, dim3((unsigned)(p.Tp / 16), (unsigned)p.nhp), dim3(256), st, aa));
  std::vector<uint8_t> hq(p.xq_bytes);
  std::vector<float> hs(p.xd_floats);
  RTQ_TRY(d2h(hq.data(), xq, p.xq_bytes, st));
  RTQ_TRY(d2h(hs.data(), xs, p.xd_floats * 4, st));
  HIP_TRY(hipStreamSynchronize(st));
  // codes of block b of token ti from the fragment layout
  const int64_t nb = K / 32, Kc = w->Kp / 128;
  auto codes = [&](int64_t ti, int64_t b, int8_t* q) {
    const int64_t kc = b / 4, j = b % 4, tg = ti / 16;
    for (int g = 0; g < 4; g++) {
      const uint8_t* f = &hq[(((tg * Kc + kc) * 4 + j) * 64 + (ti % 16) + 16 * g) * 16];
      for (int s = 0; s < 8; s++) {
        uint16_t hb;
        memcpy(&hb, f + 2 * s, 2);
        q[s < 4 ? 4 * g + s : 16 + 4 * g + (s - 4)] = (int8_t)(int)f16_bits_to_f32(hb);
      }
    }
  };
  uint8_t* o = (uint8_t*)out;
  if (!kq) {  // ggml block_q8_0: fp16 d, 32 x int8
    for (int64_t ti = 0; ti < t; ti++)
      for (int64_t b = 0; b < nb; b++) {
        uint8_t* blk = o + (ti * nb + b) * 34;
        const uint16_t d = f32_to_f16_bits(hs[((size_t)(b / 4) * p.Tp + ti) * 4 + b % 4]);  // [Kc][Tp][4]
        blk[0] = (uint8_t)(d & 0xff);
        blk[1] = (uint8_t)(d >> 8);
        codes(ti, b, (int8_t*)blk + 2);
      }
    return RTQ_OK;
  }
  // ggml block_q8_K: f32 d, 256 x int8, 16 x int16 sums of 16 codes
  const int64_t nsb = K / 256;
  for (int64_t ti = 0; ti < t; ti++)
    for (int64_t sb = 0; sb < nsb; sb++) {
      uint8_t* blk = o + (ti * nsb + sb) * 292;
      memcpy(blk, &hs[((size_t)(2 * sb) * p.Tp + ti) * 4], 4);
      int8_t* q = (int8_t*)blk + 4;
      for (int jj = 0; jj < 8; jj++) codes(ti, sb * 8 + jj, q + 32 * jj);
      for (int g = 0; g < 16; g++) {
        int16_t bs = 0;
        for (int l = 0; l < 16; l++) bs = (int16_t)(bs + q[16 * g + l]);
        memcpy(blk + 260 + 2 * g, &bs, 2);
      }
    }
  return RTQ_OK;
}

rtq_status rtq_debug_block_isums(rtq_ctx* c, const rtq_weight* w, const float* x, int64_t t, int32_t* out) {
  RTQ_TRY(check_weight(c, w));
  RTQ_TRY(check_t(t));
  if (is_dense(w->type)) return fail(RTQ_ERR_UNSUPPORTED, "trainer-native weights have no integer block sums");
  if (t == 0) return RTQ_OK;
  if (!x || !out) return fail(RTQ_ERR_INVALID, "null x/out");
  HostCall hc(c);
  HIP_TRY(hipSetDevice(c->device));
  hipStream_t st = c->stream;
  const int64_t N = w->rows, K = w->cols, m = rtq_debug_isums_per_row(w);
  FwdPlan p = fwd_plan(w, t, 0);
  const size_t isz = (size_t)(t * N * m) * 4;
  RTQ_TRY(ensure_ws(c, fwd_ws_bytes(p) + (size_t)(t * K + t * N) * 4 + isz + 4 * 256));
  Arena ar{(char*)c->ws, c->ws_bytes, 0};
  float* xdv = ar.take<float>((size_t)(t * K));
  float* yd = ar.take<float>((size_t)(t * N));
  int32_t* id = ar.take<int32_t>((size_t)(t * N * m));
  RTQ_TRY(h2d(xdv, x, (size_t)(t * K) * 4, st));
  RTQ_TRY(enqueue_forward(c, w, xdv, t, yd, nullptr, nullptr, nullptr, 0, 0.0f, id, ar, st));
  RTQ_TRY(d2h(out, id, isz, st));
  HIP_TRY(hipStreamSynchronize(st));
  return RTQ_OK;
}

}  // extern "C"

// internal (rtq_internal.h): C++ linkage, not exported as part of the C ABI
int64_t rtq_lora_partial_floats(const rtq_weight* w, int64_t t, int64_t r) {
  if (!w || is_dense(w->type) || t <= 0 || r <= 0) return 0;
  const int64_t nhp = roundup(cdiv(w->Kp, RTQ_ACT_KQ), 4);
  return nhp == lora_slices(w->cols) ? nhp * t * r : 0;  // the forward's and the backward's slicing agree
}

// a block-diagonal adapter's blocks lie inside the weight's rows and the adapter's ranks
rtq_status check_blocks(const rtq_weight* w, const rtq_lora* lora, const RankBlocks* rb) {
  if (rb && (rb->nm < 0 || rb->nm > 3)) return fail(RTQ_ERR_INVALID, "internal: %d adapter blocks", rb->nm);
  if (rb && lora && lora->enabled && lora->rank > 0) {
    for (int m = 0; m < rb->nm; m++)
      if (rb->row0[m] < 0 || rb->nrow[m] < 0 || (int64_t)rb->row0[m] + rb->nrow[m] > w->rows || rb->col0[m] < 0 ||
          rb->r[m] < 0 || (int64_t)rb->col0[m] + rb->r[m] > lora->rank)
        return fail(RTQ_ERR_INVALID, "internal: adapter block %d outside the weight or rank", m);
  }
  return RTQ_OK;
}

rtq_status rtq_linear_forward_keep_d(rtq_ctx* c, const rtq_weight* w, const float* bias, const rtq_lora* lora,
                                     const RankBlocks* rb, const float* x, int64_t t, float* y, float* hp_keep,
                                     void* stream) {
  RTQ_TRY(check_weight(c, w));
  RTQ_TRY(check_t(t));
  RTQ_TRY(check_blocks(w, lora, rb));
  bool on;
  int64_t r;
  float s;
  RTQ_TRY(check_lora(lora, &on, &r, &s));
  if (t > 0 && (!x || !y)) return fail(RTQ_ERR_INVALID, "null x/y");
  if (hp_keep && rtq_lora_partial_floats(w, t, on ? r : 0) == 0) hp_keep = nullptr;
  std::lock_guard<std::mutex> lk(c->mu);
  HIP_TRY(hipSetDevice(c->device));
  hipStream_t st = (hipStream_t)stream;
  FwdPlan p = fwd_plan(w, t, on ? r : 0);
  RTQ_TRY(ensure_ws(c, fwd_ws_bytes(p)));
  Arena ar{(char*)c->ws, c->ws_bytes, 0};
  return enqueue_forward(c, w, x, t, y, bias, on ? lora->a : nullptr, on ? lora->b : nullptr, r, s, nullptr, ar, st,
                         hp_keep, rb);
}

rtq_status rtq_linear_forward_swiglu_d(rtq_ctx* c, const rtq_weight* w, const float* bias, const rtq_lora* lora,
                                       const RankBlocks* rb, const float* g, const float* u, int64_t ldg,
                                       float* x_out, int64_t t, float* y, float* hp_keep, void* stream) {
  RTQ_TRY(check_weight(c, w));
  RTQ_TRY(check_t(t));
  RTQ_TRY(check_blocks(w, lora, rb));
  if (is_dense(w->type)) return fail(RTQ_ERR_UNSUPPORTED, "SwiGLU input: quantised weights only");
  bool on;
  int64_t r;
  float s;
  RTQ_TRY(check_lora(lora, &on, &r, &s));
  if (t > 0 && (!g || !u || !x_out || !y)) return fail(RTQ_ERR_INVALID, "null g/u/x/y");
  if (ldg < w->cols || ldg % 4 != 0 || ((uintptr_t)g | (uintptr_t)u | (uintptr_t)x_out) % 16 != 0)
    return fail(RTQ_ERR_INVALID, "SwiGLU input: rows of at least cols floats, 16-byte aligned");
  if (hp_keep && rtq_lora_partial_floats(w, t, on ? r : 0) == 0) hp_keep = nullptr;
  std::lock_guard<std::mutex> lk(c->mu);
  HIP_TRY(hipSetDevice(c->device));
  hipStream_t st = (hipStream_t)stream;
  FwdPlan p = fwd_plan(w, t, on ? r : 0);
  RTQ_TRY(ensure_ws(c, fwd_ws_bytes(p)));
  Arena ar{(char*)c->ws, c->ws_bytes, 0};
  const SwiGluIn sw{g, u, ldg};
  return enqueue_forward(c, w, x_out, t, y, bias, on ? lora->a : nullptr, on ? lora->b : nullptr, r, s, nullptr, ar,
                         st, hp_keep, rb, &sw);
}

bool rtq_norm_fusable(const rtq_weight* w, const NormIn& n, const float* x_out) {
  return w && !is_dense(w->type) && w->cols % 256 == 0 && w->cols <= 1024 && n.a && n.w && n.inv && x_out &&
         (!n.b || n.h) && ((uintptr_t)n.a | (uintptr_t)n.b | (uintptr_t)n.h | (uintptr_t)n.w | (uintptr_t)x_out) % 16 == 0;
}

rtq_status rtq_linear_forward_norm_d(rtq_ctx* c, const rtq_weight* w, const float* bias, const rtq_lora* lora,
                                     const RankBlocks* rb, const NormIn* n, float* x_out, int64_t t, float* y,
                                     float* hp_keep, void* stream) {
  RTQ_TRY(check_weight(c, w));
  RTQ_TRY(check_t(t));
  RTQ_TRY(check_blocks(w, lora, rb));
  if (!n || !rtq_norm_fusable(w, *n, x_out))
    return fail(RTQ_ERR_UNSUPPORTED, "norm input: quantised weights, cols %% 256 == 0 and <= 1024, 16-byte aligned rows");
  bool on;
  int64_t r;
  float s;
  RTQ_TRY(check_lora(lora, &on, &r, &s));
  if (t > 0 && !y) return fail(RTQ_ERR_INVALID, "null y");
  if (hp_keep && rtq_lora_partial_floats(w, t, on ? r : 0) == 0) hp_keep = nullptr;
  std::lock_guard<std::mutex> lk(c->mu);
  HIP_TRY(hipSetDevice(c->device));
  hipStream_t st = (hipStream_t)stream;
  FwdPlan p = fwd_plan(w, t, on ? r : 0);
  RTQ_TRY(ensure_ws(c, fwd_ws_bytes(p)));
  Arena ar{(char*)c->ws, c->ws_bytes, 0};
  return enqueue_forward(c, w, x_out, t, y, bias, on ? lora->a : nullptr, on ? lora->b : nullptr, r, s, nullptr, ar,
                         st, hp_keep, rb, nullptr, n);
}

rtq_status rtq_linear_forward_ws_d(rtq_ctx* c, const rtq_weight* w, const float* bias, const rtq_lora* lora,
                                   const float* x, int64_t t, float* y, void* stream, void* ws, size_t ws_bytes) {
  RTQ_TRY(check_weight(c, w));
  RTQ_TRY(check_t(t));
  bool on;
  int64_t r;
  float s;
  RTQ_TRY(check_lora(lora, &on, &r, &s));
  if (t > 0 && (!x || !y)) return fail(RTQ_ERR_INVALID, "null x/y");
  const size_t need = fwd_ws_bytes(fwd_plan(w, t, on ? r : 0));
  if (need > ws_bytes)
    return fail(RTQ_ERR_INVALID, "forward of %lld tokens over %lldx%lld needs %zu bytes of scratch; the maximum is %zu",
                (long long)t, (long long)w->rows, (long long)w->cols, need, ws_bytes);
  std::lock_guard<std::mutex> lk(c->mu);
  HIP_TRY(hipSetDevice(c->device));
  Arena ar{(char*)ws, ws_bytes, 0};
  return enqueue_forward(c, w, x, t, y, bias, on ? lora->a : nullptr, on ? lora->b : nullptr, r, s, nullptr, ar,
                         (hipStream_t)stream);
}

rtq_status rtq_linear_backward_defer_d(rtq_ctx* c, const rtq_weight* w, const rtq_lora* lora, const RankBlocks* rb,
                                       const float* x, const float* dy, int64_t t, float* dx, float* ga, float* gb,
                                       const float* hp_have, float* h_out, float* g_out, LoraGradArgs* job,
                                       void* stream, const SwiGluBwd* sw) {
  RTQ_TRY(check_weight(c, w));
  RTQ_TRY(check_blocks(w, lora, rb));
  if (!job || !h_out || !g_out) return fail(RTQ_ERR_INVALID, "deferred backward needs h, g and a job");
  if (sw && (!sw->g || !sw->u || !sw->dg || !sw->du || sw->ld < w->cols))
    return fail(RTQ_ERR_INVALID, "SwiGLU backward: null g/u/dg/du or rows shorter than cols");
  if (is_dense(w->type)) return fail(RTQ_ERR_INVALID, "deferred backward: quantised weights only");
  if (hp_have && rtq_lora_partial_floats(w, t, lora && lora->enabled ? lora->rank : 0) == 0) hp_have = nullptr;
  const LoraDefer df{h_out, g_out, job, sw};
  return linear_backward_d(c, w, lora, x, dy, t, dx, ga, gb, stream, rb, hp_have, &df);
}

rtq_status rtq_lora_grads_d(rtq_ctx* c, const LoraGradArgs* jobs, int n, void* stream) {
  if (!c) return fail(RTQ_ERR_INVALID, "null context");
  if (n < 0 || n > RTQ_LORA_JOBS) return fail(RTQ_ERR_INVALID, "%d LoRA gradient jobs (at most %d)", n, RTQ_LORA_JOBS);
  LoraGradBatch b{};
  int64_t total = 0, tmax = 0;
  for (int i = 0; i < n; i++) {
    if (jobs[i].n_gb + jobs[i].n_ga == 0) continue;
    b.start[b.njobs] = (int)total;
    b.job[b.njobs++] = jobs[i];
    total += jobs[i].n_gb + jobs[i].n_ga;
    tmax = std::max<int64_t>(tmax, jobs[i].T);
  }
  b.start[b.njobs] = (int)total;
  if (total == 0) return RTQ_OK;
  std::lock_guard<std::mutex> lk(c->mu);
  HIP_TRY(hipSetDevice(c->device));
  const bool w16 = tmax >= 256;  // 16 waves split long token ranges, as in rtq_bwd_finish16
  return launch(c, w16 ? K_LORA_GRADS16 : K_LORA_GRADS, dim3((unsigned)total), dim3(w16 ? 1024 : 256),
                (hipStream_t)stream, b);
}

rtq_status rtq_lora_grads_table_d(rtq_ctx* c, const LoraGradArgs* jobs_d, const int* map_d, int64_t nwg, bool w16,
                                  void* stream) {
  if (!c) return fail(RTQ_ERR_INVALID, "null context");
  if (nwg <= 0) return RTQ_OK;
  if (!jobs_d || !map_d || nwg > INT32_MAX) return fail(RTQ_ERR_INVALID, "LoRA gradient table: null or too large");
  std::lock_guard<std::mutex> lk(c->mu);
  HIP_TRY(hipSetDevice(c->device));
  const LoraGradTable tb{jobs_d, map_d};
  return launch(c, w16 ? K_LORA_GRADS_T16 : K_LORA_GRADS_T, dim3((unsigned)nwg), dim3(w16 ? 1024 : 256),
                (hipStream_t)stream, tb);
}

rtq_status rtq_linear_backward_blocks_d(rtq_ctx* c, const rtq_weight* w, const rtq_lora* lora, const RankBlocks* rb,
                                        const float* x, const float* dy, int64_t t, float* dx, float* ga, float* gb,
                                        const float* hp_have, void* stream) {
  RTQ_TRY(check_weight(c, w));
  RTQ_TRY(check_blocks(w, lora, rb));
  if (hp_have && rtq_lora_partial_floats(w, t, lora && lora->enabled ? lora->rank : 0) == 0) hp_have = nullptr;
  return linear_backward_d(c, w, lora, x, dy, t, dx, ga, gb, stream, rb, hp_have);
}
