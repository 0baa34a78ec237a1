// rtq_internal.h — declarations shared by the translation units of librtq.so (not part of the
// C ABI): error reporting and kernel launches by the model-level step (rtq_model.cpp).
#ifndef RTQ_INTERNAL_H
#define RTQ_INTERNAL_H
#include <hip/hip_runtime.h>

#include "rtq.h"
#include "rtq_kargs.h"

// kernels of the decoder block (rtq_model_kernels.hip), in this order after the matmul kernels
enum RtqModelKernel {
  KM_RMSNORM,
  KM_RMSNORM_BWD,
  KM_QK_PREP,
  KM_QK_BWD,
  KM_GEMM,
  KM_SOFTMAX,
  KM_SOFTMAX_BWD,
  KM_GROUP_SUM,
  KM_SWIGLU,
  KM_SWIGLU_BWD,
  KM_ADD,
  KM_GEMM32,
  KM_LORA_MASK,
  KM_GEMM32G,
  KM_GEMM_Q8,
  KM_GEMM32_Q8,
  KM_ATTN_MERGE_FWD,
  KM_ATTN_MERGE_BWD,
  KM_ATTN_BWD_PREP64,  // the fused backward's operand planes and D = dO . o (head size 64, 128)
  KM_GEMM_BF,
  KM_GEMM32_BF,
  KM_GEMM32G_BF,
  KM_GEMM_HF,
  KM_GEMM32_HF,
  KM_FA_FWD64,
  KM_FA_FWD128,
  KM_FA_BWD64,
  KM_FA_BWD128,
  KM_ATTN_BWD_PREP128,
  KM_SEQ_GATHER,  // the forward attention of a packed layout over each segment's logical sequence
  KM_SEQ_SCATTER,
  KM_COUNT
};

// sets the thread-local message of rtq_last_error and returns st
rtq_status rtq_fail(rtq_status st, const char* fmt, ...);
// launches decoder kernel km with one by-value argument struct at args (timed like every launch)
rtq_status rtq_model_launch(rtq_ctx* c, int km, dim3 grid, dim3 block, hipStream_t s, const void* args);
int rtq_ctx_device_id(const rtq_ctx* c);
int rtq_ctx_cu_count(const rtq_ctx* c);
// generation of the context's workspace (changes whenever it is reallocated)
uint64_t rtq_ctx_ws_gen(const rtq_ctx* c);
// per-launch timing is on (rtq_ctx_set_timing): launches record events
bool rtq_ctx_timing_on(const rtq_ctx* c);
// floats of the LoRA-down partials a forward of t tokens at rank r can keep for the backward of the
// same x (0: not kept for this weight - dense, or slicings that differ)
int64_t rtq_lora_partial_floats(const rtq_weight* w, int64_t t, int64_t r);
// rtq_linear_forward_d that also leaves the LoRA-down partials in hp_keep (null or too small a
// weight: as rtq_linear_forward_d); rb (or null): the adapter's block-diagonal structure, so each
// row's up-projection reads its own member's ranks only (B is zero elsewhere)
rtq_status rtq_linear_forward_keep_d(rtq_ctx* c, const rtq_weight* w, const float* bias, const rtq_lora* lora,
                                     const RankBlocks* rb, const float* x, int64_t t, float* y, float* hp_keep,
                                     void* stream);
// rtq_linear_forward_keep_d of x = silu(g) * u (SwiGLU, src/model.rs:124; g and u rows of stride
// ldg floats, 16-byte aligned): the activation kernel forms x and writes it to x_out [t x cols] for
// the backward.  Quantised weights only (a dense one: RTQ_ERR_UNSUPPORTED, the caller forms x).
rtq_status rtq_linear_forward_swiglu_d(rtq_ctx* c, const rtq_weight* w, const float* bias, const rtq_lora* lora,
                                       const RankBlocks* rb, const float* g, const float* u, int64_t ldg,
                                       float* x_out, int64_t t, float* y, float* hp_keep, void* stream);
// rtq_linear_forward_keep_d of x = RMSNorm(a (+ b)) (src/ops.rs:14-35: (x / rms) (w + off), the
// one-wave row order of the model's norm kernel): the activation kernel forms the rows and writes
// them to x_out [t x cols], a + b to h (with b) and 1 / rms to inv [t].  Quantised weights with
// cols % 256 == 0, cols <= 1024 and 16-byte aligned rows (else RTQ_ERR_UNSUPPORTED: the caller
// normalises first).
struct NormIn {
  const float* a;
  const float* b;  // or null
  float* h;        // a + b (with b)
  const float* w;
  float* inv;
  float eps, off;
};
bool rtq_norm_fusable(const rtq_weight* w, const NormIn& n, const float* x_out);
rtq_status rtq_linear_forward_norm_d(rtq_ctx* c, const rtq_weight* w, const float* bias, const rtq_lora* lora,
                                     const RankBlocks* rb, const NormIn* n, float* x_out, int64_t t, float* y,
                                     float* hp_keep, void* stream);
// rtq_linear_backward_d for a block-diagonal adapter over row-concatenated weights (rb; null: a
// plain adapter): gb and g = s dy.B only inside rb's blocks (gb outside them is left untouched).
// Quantised weights only; a dense weight computes every pair (the caller clears gb outside the
// blocks).  hp_have: the partials a rtq_linear_forward_keep_d of the same x left (or null).
rtq_status rtq_linear_backward_blocks_d(rtq_ctx* c, const rtq_weight* w, const rtq_lora* lora, const RankBlocks* rb,
                                        const float* x, const float* dy, int64_t t, float* dx, float* ga, float* gb,
                                        const float* hp_have, void* stream);
// rtq_linear_backward_blocks_d whose dA / dB are not launched but described in *job, for one
// rtq_lora_grads_d over several linears; h and g are written to h_out / g_out ([t x r] each), which,
// like x, dy, ga and gb, must stay untouched until that launch has run (quantised weights only)
// sw (or null): dx is SwiGLU's dh (src/model.rs:126-131); it is not stored, the dx kernels' finish
// writes dg = (dh u) silu'(g) and du = dh silu(g) instead (rows of stride ld)
struct SwiGluBwd {
  const float* g;
  const float* u;
  float* dg;
  float* du;
  int64_t ld;
  bool keep_dh;  // dh is stored to dx as well
};
rtq_status rtq_linear_backward_defer_d(rtq_ctx* c, const rtq_weight* w, const rtq_lora* lora, const RankBlocks* rb,
                                       const float* x, const float* dy, int64_t t, float* dx, float* ga, float* gb,
                                       const float* hp_have, float* h_out, float* g_out, LoraGradArgs* job,
                                       void* stream, const SwiGluBwd* sw = nullptr);
// dA / dB of n (<= RTQ_LORA_JOBS) deferred linears in one launch (jobs with no tiles are skipped)
rtq_status rtq_lora_grads_d(rtq_ctx* c, const LoraGradArgs* jobs, int n, void* stream);
// the dA / dB tiles of a job table already in device memory: workgroup b runs tile map_d[2 b + 1] of
// job map_d[2 b] (nwg workgroups; w16: 16 waves per workgroup, for token counts of 256 and more)
rtq_status rtq_lora_grads_table_d(rtq_ctx* c, const LoraGradArgs* jobs_d, const int* map_d, int64_t nwg, bool w16,
                                  void* stream);
// rtq_noalloc.hip: resolves the no-allocation scratch array's address on `device` (current)
rtq_status rtq_scratch_setup(int device);
// rtq_linear_forward_d with the caller's workspace ws (ws_bytes) instead of the context's: never
// allocates; a forward needing more than ws_bytes fails with RTQ_ERR_INVALID before any launch.
rtq_status rtq_linear_forward_ws_d(rtq_ctx* c, const rtq_weight* w, const float* bias, const rtq_lora* lora,
                                   const float* x, int64_t t, float* y, void* stream, void* ws, size_t ws_bytes);
#endif
