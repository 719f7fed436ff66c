/*
 * oracle.h — CPU restatement of SharpMind's training-path kernels.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the sharpmind_amd
 * package, libsharpmind_hip.so) may link, load or call this code.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it,
 * and only as the checker / the timed CPU baseline.
 *
 * Each function cites the reference file:line it restates (paths relative
 * to the SharpMind repository root).  Loop order and precision follow the
 * reference: float arithmetic where C# uses float, double where C# uses
 * double, no FMA contraction (the file is compiled with -ffp-contract=off).
 */
#ifndef SHARPMIND_ORACLE_H
#define SHARPMIND_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- .NET System.Random(seed) (legacy seeded Knuth subtractive generator) */
typedef struct { int32_t seed[56]; int inext, inextp; } orc_rng;
void   orc_rng_init(orc_rng* r, int32_t seed);
int32_t orc_rng_sample(orc_rng* r);              /* InternalSample()         */
double orc_rng_next_double(orc_rng* r);          /* NextDouble()             */
void   orc_rng_next_bytes(orc_rng* r, uint8_t* buf, int64_t n);
/* WeightInitializer.FillNormal (SharpMind.Training/WeightInitializer.cs:98-106) */
void   orc_fill_normal(orc_rng* r, float* data, int64_t n, float std);
/* convenience: fill n doubles via NextDouble()*2-1 as float (VecDotTests.cs:524-590) */
void   orc_fill_uniform_pm1(orc_rng* r, float* data, int64_t n);

/* ---- half <-> float */
float    orc_half_to_float(uint16_t h);          /* QuantizationKernels.cs:117-146 */
uint16_t orc_float_to_half_rne(float f);         /* (Half)f, QuantizationKernels.cs:149 */

/* ---- Q8_0 / Q4_K (block layouts: QuantizationOps.cs:37, QuantizationKernels.Q4.cs:586-624) */
void  orc_dequant_q8_0(const uint8_t* raw, float* out, int64_t n);   /* ReadQ8_0_Scalar Q8.cs:412-433 */
void  orc_dequant_q4k(const uint8_t* raw, float* out, int64_t n);    /* ReadQ4K_Scalar Q4.cs:951-981 */
float orc_vecdot_q8_0(const float* in, const uint8_t* raw, int col, int K); /* Q8.cs:11-26 */
float orc_vecdot_q4k(const float* in, const uint8_t* raw, int col, int K);  /* Q4.cs:586-624 */
/* QuantizedMatMulFn semantics: out[m,n] = vecdot(in row m, W col n) (Q8.cs:556-573) */
void  orc_qmatmul_q8_0(const float* in, const uint8_t* raw, float* out, int M, int K, int N);
void  orc_qmatmul_q4k(const float* in, const uint8_t* raw, float* out, int M, int K, int N);
void  orc_qmatmul_f32(const float* in, const float* w, float* out, int M, int K, int N);
/* encoders: TensorQuantizer.cs:80-144 (Q8_0), TensorQuantizer.KQuant.cs:173-225,451-459 (Q4_K) */
int   orc_quantize_q8_0(const float* x, int64_t n, uint8_t* out);
int   orc_quantize_q4k(const float* x, int64_t n, uint8_t* out);

/* ---- GradientMapping slots (SharpMind.Core/Training/Kernels/GradientKernels.cs) */
/* Linear_Scalar :50-112.  W [Out,In]; dX overwritten; dW += ; db += (nullable) */
void orc_grad_linear(const float* dY, const float* X, const float* W, float* dW, float* db,
                     float* dX, int B, int In, int Out);
/* RMSNorm_Scalar :303-337 */
void orc_grad_rmsnorm(const float* dY, const float* xNorm, const float* rmsInv, const float* w,
                      float* dw, float* dX, int T, int D);
/* LayerNorm_Scalar :345-398 */
void orc_grad_layernorm(const float* dY, const float* x, const float* w, float* dw, float* db,
                        float* dX, int T, int D, float eps);
/* Attention_Scalar :408-481 (one head; dQ/dK/dV overwritten) */
void orc_grad_attention(const float* dO, const float* q, const float* k, const float* v,
                        const float* probs, float* dQ, float* dK, float* dV, int S, int D, float scale);
/* Embedding_Scalar :490-506 */
void orc_grad_embedding(const float* dY, const int32_t* ids, float* dE, int T, int D);
/* ActivationSiLU_Scalar :559-573, ActivationGELU_Scalar :612-630 */
void orc_grad_silu(const float* dY, const float* x, float* dX, int64_t n);
void orc_grad_gelu(const float* dY, const float* x, float* dX, int64_t n);

/* ---- inline BackpropEngine pieces (SharpMind.Training/Autograd/BackpropEngine.cs) */
/* SwiGLU backward :623-657 with GateValue/GateDerivative :859-884 (SiLU);
 * writes the fused [dGate | dUp] row layout [T, 2F]. */
void orc_grad_swiglu(const float* dAct, const float* gate, const float* up, float* dFused, int T, int F);
/* SwiGLU forward, scalar tier (ActivationKernels.cs:194-205) */
void orc_swiglu_fwd(const float* gate, const float* up, float* act, int64_t n);

/* ---- RoPE (SharpMind.Core/Embeddings/RoPE.cs) */
/* tables :99-148 (no scaling): cos/sin [maxSeq, ropeDim/2] */
void orc_rope_tables(float theta, int ropeDim, int maxSeq, float* cosT, float* sinT);
/* Apply :168-259 on x [S, H, D] (one batch slice) */
void orc_rope_fwd(float* x, const float* cosT, const float* sinT, int S, int H, int D, int neox);
/* ApplyBackward :300-347 */
void orc_rope_bwd(float* dx, const float* cosT, const float* sinT, int S, int H, int D, int neox);

/* ---- RMSNorm forward (NormKernels.cs:40-60 rmsInv, :13-33 row apply) */
float orc_rmsnorm_param(const float* row, int n, float eps);
void  orc_rmsnorm_fwd(const float* x, const float* w, float* y, float* rmsInv, int T, int D, float eps);

/* ---- loss (SharpMind.Training/Autograd/Gradients.cs:33-84, Loss/CrossEntropyLoss.cs:44-104) */
void  orc_ce_softmax_grad(const float* logits, const int32_t* labels, float* dLogits, int T, int V,
                          int ignoreId, float smoothing);
float orc_ce_loss(const float* logits, const int32_t* labels, int T, int V, int ignoreId, float smoothing);

/* ---- TrainingOps (SharpMind.Training/TrainingKernels.cs) */
void  orc_adamw(float* data, const float* grad, float* m, float* v, int64_t n, float beta1, float beta2,
                float bc1, float bc2, float lr, float eps, float decay);          /* :75-89 */
float orc_l2normsq(const float* data, int64_t n);                                 /* :129-134 */

/* ---- causal attention forward, exact-exp scalar path (BackpropEngine.cs:237-388)
 * q [B,S,Hq,D], k/v [B,S,Hkv,D] -> probs [B,Hq,S,S] (zeros above diagonal), out [B,S,Hq*D] */
void orc_attention_fwd(const float* q, const float* k, const float* v, float* probs, float* out,
                       int B, int S, int Hq, int Hkv, int D);

/* ---- LoRA (math contract of LoRALayer.Forward, SharpMind.Training/LoRA/LoRALayer.cs:52-80)
 * y = x W^T + s (x A) B ; A [In,r], B [r,Out].  Backward (no reference implementation):
 * dB += s (xA)^T dY ; dA += s x^T (dY B^T) ; dX = dY W + s (dY B^T) A^T   (all in double) */
void orc_lora_fwd(const float* x, const float* W, const float* A, const float* Bm, float* y,
                  int T, int In, int Out, int r, float s);
void orc_lora_bwd(const float* dY, const float* x, const float* W, const float* A, const float* Bm,
                  float* dA, float* dB, float* dX, int T, int In, int Out, int r, float s);

#ifdef __cplusplus
}
#endif
#endif
