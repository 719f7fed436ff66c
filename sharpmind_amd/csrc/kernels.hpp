// kernels.hpp — internal launchers shared between translation units.
#pragma once
#include "common.hpp"

namespace smhip {

// elementwise.hip
int rmsnorm_backward(const float* dY, const float* xin, int from_x, const float* rinv,
                     const float* w, float* dw, float* dX, int T, int D, int accumulate,
                     uint16_t* dX_bf16, hipStream_t s);
int rmsnorm_forward(const float* x, const float* w, float* y, uint16_t* yb, float* rinv, int T,
                    int D, float eps, hipStream_t s);
int layernorm_backward(const float* dY, const float* x, const float* w, float* dw, float* db,
                       float* dX, int T, int D, float eps, hipStream_t s);
int swiglu_backward_f32(const float* dAct, const float* gate, const float* up, float* dFused, int T,
                        int F, hipStream_t s);
int swiglu_backward_mixed(const float* dAct, const uint16_t* gu, uint16_t* dgu, int T, int F,
                          hipStream_t s);
int swiglu_forward_f32(const float* g, const float* u, float* a, int64_t n, hipStream_t s);
int swiglu_forward_bf16(const uint16_t* gu, uint16_t* act, int T, int F, hipStream_t s);
int silu_backward(const float* dy, const float* x, float* dx, int64_t n, hipStream_t s);
int gelu_backward(const float* dy, const float* x, float* dx, int64_t n, hipStream_t s);
int rope_apply(float* x, const float* cosT, const float* sinT, int B, int S, int H, int D, int neox,
               int backward, hipStream_t s);
int ce_softmax_grad(const float* logits, const int32_t* labels, float* dL, float* loss, int T, int V,
                    int ignoreId, float smoothing, hipStream_t s);
int ce_softmax_grad_bf16(const float* logits, const int32_t* labels, uint16_t* dL, float* loss,
                         int T, int V, int ignoreId, float smoothing, hipStream_t s);
// the same with the row statistics precomputed by the logits' GEMM ([T][nst] (max, sum exp)
// pairs over consecutive column blocks): the logits are read once; no label smoothing
int ce_softmax_grad_bf16_stats(const float* logits, const float* stats, int nst, const int32_t* labels, uint16_t* dL,
                               float* loss, int T, int V, int ignoreId, hipStream_t s);
// shadow: optional bf16 copy of the updated parameters; clip_nsq: optional device sum of squares
// of the whole gradient -- when sqrt(*clip_nsq) > clip_max the gradient is first scaled by
// clip_max / sqrt(*clip_nsq) (and stored back scaled), as a separate clip pass would
int adamw_update(float* data, const float* grad, float* m, float* v, int64_t n, float b1, float b2,
                 float bc1, float bc2, float lr, float eps, float decay, hipStream_t s, uint16_t* shadow = nullptr,
                 const float* clip_nsq = nullptr, float clip_max = 0.f);
int l2normsq(const float* x, int64_t n, float* out, int accumulate, hipStream_t s);
int scale_inplace(float* x, int64_t n, float sc, hipStream_t s);
int embedding_backward(const float* dY, const int32_t* ids, float* dE, int T, int D, int V,
                       hipStream_t s);
int embedding_forward(const float* E, const int32_t* ids, float* out, int T, int D, hipStream_t s);
int add_inplace(float* y, const float* x, int64_t n, hipStream_t s);
int f32_to_bf16(const float* x, uint16_t* y, int64_t n, hipStream_t s);
int colsum_add(const float* dY, float* db, int B, int Out, hipStream_t s);

// gemm_bf16.hip: 1 = ran, 0 = not eligible (generic kernel), <0 = error
int gemm_bf16_fast(const GemmArgs& g, hipStream_t s);
// Deferred split reductions of rank-sized products: gemm_skinny with a batch writes its fp32
// partials into the batch's arena and queues the reduction; skinny_flush reduces everything
// queued in one launch (also called by gemm_skinny when the arena or the queue is full).
// Products whose result is not read before the flush (gradient accumulations) may be deferred.
// Block-diagonal output mask of a fused LoRA B gradient (dB^T stored transposed, rows r of n,
// columns m of M): entry (r, m) is written only when cols[r / rank] <= m < cols[r / rank + 1]
// (M for the last block); the others keep their value (zero: gradients are cleared per step).
struct SkinnyMask {
  const int* cols = nullptr;  // device, nblk column starts; nullptr: no mask
  int rank = 0, nblk = 0;
};
struct SkinnyJob {
  const float* partial;
  void* C;
  int64_t ldc;
  int S, M, n;
  float alpha, beta;
  int trans, c_bf16;
  SkinnyMask mask;
};
struct SkinnyBatch {
  static constexpr int kMaxJobs = 8;
  float* arena = nullptr;
  size_t cap = 0, used = 0;  // bytes
  int n = 0;
  SkinnyJob job[kMaxJobs];
};
int skinny_flush(SkinnyBatch* b, hipStream_t s);
// A rank-sized product whose launch is held back so the next compatible one (same operand kinds,
// rank and output type) shares its launch.  skinny_release launches whatever is still held.
struct SkinnyHold {
  bool valid = false;
  bool big_k, small_k, trans, c_bf16;
  int mt, S, n, M, K;
  unsigned char args[256];  // the product's kernel arguments (sk::Args)
};
int skinny_release(SkinnyHold* h, hipStream_t s);
// batched bf16 transposes: dst [cols][rows] = src [rows][cols] for each job (one launch)
struct BfTJob {
  const uint16_t* src;
  uint16_t* dst;
  int rows, cols;
};
int transpose_bf16_jobs(const BfTJob* jobs_dev, int njobs, int64_t max_elems, hipStream_t s);
// SwiGLU forward (bf16 [gate | up] in, bf16 act out) fused with u = act A for a LoRA A given
// transposed, At [n][F] (bf16); 1 = done, 0 = shapes unsupported (run them separately)
int swiglu_lora_u(const uint16_t* gu, uint16_t* act, const uint16_t* At, int n, uint16_t* u, int T, int F,
                  hipStream_t s);
// RMSNorm forward (bf16 output) fused with u = xn A for a LoRA A given transposed, At [n][D] (bf16); 1 = done, 0 = shape
// not supported (run rmsnorm_forward and the rank product instead)
int rmsnorm_lora_u(const float* h, const float* w, float eps, uint16_t* xn, float* rinv, const uint16_t* At, int n,
                   uint16_t* u, int T, int D, hipStream_t s);
int gemm_skinny(int M, int n, int K, const void* big, int64_t ldb, bool big_k, const void* small, int64_t lds,
                bool small_k, float alpha, float beta, void* C, int64_t ldc, bool trans_out, bool c_bf16,
                SkinnyBatch* defer, hipStream_t s, SkinnyMask mask = SkinnyMask{}, SkinnyHold* hold = nullptr);

// quant.hip
int dequant_raw(int qtype, const void* raw, float* out, int64_t n, hipStream_t s);
size_t planes_bytes(int qtype, int64_t n, size_t* qs_bytes);
int repack_planes(int qtype, const void* raw, int64_t n, void* dst, QuantPlanes* out, hipStream_t s);
int dequant_rows(const QuantPlanes& q, const int32_t* ids, float* out, int T, int D, hipStream_t s);
int make_col_planes(const QuantPlanes& q, int rows, int cols, void* dst, QuantPlanes* out, hipStream_t s);
// fragment planes (SRC_Q8F / SRC_Q4F for trans = 0: B = W; SRC_Q8FT / SRC_Q4FT for trans = 1:
// B = W^T) of Q8_0 or Q4_K row planes of W[rows][cols] into dst (frag_planes_bytes(rows*cols,
// qtype) bytes, 256-byte aligned)
size_t frag_planes_bytes(int64_t n, int qtype);
int make_frag_planes(const QuantPlanes& q, int rows, int cols, int trans, void* dst, Operand* out, hipStream_t s);
// one launch decoding many matrices; `first` = index of the job's first 64x64 tile in the grid
struct DequantJob {
  QuantPlanes q;
  int rows, cols;
  uint16_t* w;
  uint16_t* wt;
  int64_t first;
};
int dequant_bf16_check(const QuantPlanes& q, int rows, int cols, const uint16_t* w, const uint16_t* wt);
int dequant_bf16_many(const DequantJob* jobs_dev, int njobs, int64_t total_tiles, hipStream_t s);

// attention.hip
int attention_slot_backward(const float* dO, const float* q, const float* k, const float* v,
                            const float* P, float* dQ, float* dK, float* dV, int S, int D,
                            float scale, hipStream_t s);
int attention_forward_probs(const float* q, const float* k, const float* v, float* probs, float* out,
                            int B, int S, int Hq, int Hkv, int D, hipStream_t s);

}  // namespace smhip

namespace smhip {
// flash.hip
int flash_forward(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o, float* lse, int B,
                  int S, int Hq, int Hkv, int D, int64_t ldq, int64_t ldk, int64_t ldv, int64_t ldo,
                  hipStream_t s);
size_t flash_backward_workspace(int B, int S, int Hq, int D);
// dk == dv == nullptr: flash_backward leaves the per-query-head partials dK_h, dV_h [B*S, Hq, D]
// in the workspace instead of summing each GQA group; these are their addresses.  bf16_grads:
// dq and the partials are bf16 (requires dk == dv == nullptr), fp32 otherwise.
void flash_backward_partials(void* ws, int B, int S, int Hq, int D, const void** dKh, const void** dVh);
int flash_backward(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* o,
                   const uint16_t* dO, const float* lse, void* dq, float* dk, float* dv, int B, int S,
                   int Hq, int Hkv, int D, int64_t ldq, int64_t ldk, int64_t ldv, int64_t ldo, int64_t lddo,
                   int64_t lddq, int64_t lddk, int64_t lddv, void* ws, hipStream_t s, int bf16_grads = 0);
// attention.hip (probability-materialising path, head-strided)
int attention_probs_backward(const float* dO, const float* q, const float* k, const float* v,
                             const float* probs, float* dq, float* dk, float* dv, int B, int S, int Hq,
                             int Hkv, int D, hipStream_t s);
// engine_kernels.hip
int qkv_prep_forward(const void* qkv, int qkv_bf16, void* q, void* k, void* v, float* rinv, const float* wq,
                     const float* wk, const float* cosT, const float* sinT, int T, int S, int Hq, int Hkv,
                     int D, int qk_norm, int neox, float eps, int bf16, hipStream_t s);
int qkv_prep_backward(const void* dq, const void* dk, const void* dv, int grads_bf16, const void* qkv, int qkv_bf16,
                      const float* rinv,
                      const float* wq, const float* wk, float* dwq, float* dwk, const float* cosT,
                      const float* sinT, void* dqkv, int T, int S, int Hq, int Hkv, int D, int qk_norm,
                      int neox, int bf16, int kv_grp, hipStream_t s);
int swiglu_fused_forward(const void* gu, void* act, int T, int F, int bf16, hipStream_t s);
int swiglu_fused_backward(const void* dA, const void* gu, void* dgu, int T, int F, int bf16, hipStream_t s);
int lora_mask(float* dB, int nr, int r, int Out, const int* col_starts_dev, int nblocks, hipStream_t s);
int cast_bf16(const float* x, uint16_t* y, int64_t n, hipStream_t s);
int fill_normal(float* x, int64_t n, uint64_t seed, float mean, float std, hipStream_t s);
int fill_uniform(float* x, int64_t n, uint64_t seed, float lo, float hi, hipStream_t s);
int fill_ids(int32_t* x, int64_t n, uint64_t seed, int V, hipStream_t s);
int encode_quant(int qtype, const float* x, int64_t n, void* out, hipStream_t s);
int zero_bytes(void* p, size_t bytes, hipStream_t s);
}  // namespace smhip
