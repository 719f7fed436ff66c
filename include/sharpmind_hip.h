/*
 * sharpmind_hip.h — C ABI of libsharpmind_hip, the MI355X (gfx950) backward-pass
 * backend for SharpMind's autograd training stack.
 *
 * Conventions
 *  - Every entry returns int: SMHIP_OK (0) or a negative SMHIP_E* code; the
 *    message is available from smhip_last_error() on the calling thread.
 *  - "Device" entries take device pointers (hipMalloc'd memory) and an explicit
 *    stream (hipStream_t passed as void*, NULL = the default stream).  They are
 *    asynchronous.  "smhip_host_*" entries take host pointers, copy in/out and
 *    synchronise; they are the drop-in parity path for the C# P/Invoke shim.
 *  - All matrices are row-major.  Parameter gradients are ACCUMULATED (+=),
 *    returned activations gradients (dX) are OVERWRITTEN, exactly as the
 *    reference's GradientMapping contract (SharpMind.Core/Training/
 *    GradientMapping.cs:7-16).
 *  - Thread safety: entries are re-entrant.  Internal scratch is keyed by stream;
 *    device entries issued concurrently from several threads must use distinct streams.
 *    smhip_host_* entries run on a stream (and scratch) private to the calling thread, so
 *    they may be called concurrently, as the reference's Parallel.For bodies call its slots
 *    (BackpropEngine.cs:563-582).
 */
#ifndef SHARPMIND_HIP_H
#define SHARPMIND_HIP_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SMHIP_OK 0
#define SMHIP_EINVAL (-1)
#define SMHIP_EHIP (-2)
#define SMHIP_ENOMEM (-3)
#define SMHIP_EUNSUPPORTED (-4)

/* GEMM arithmetic: fp32 MFMA (exactness mode) or bf16 MFMA with fp32 accumulate. */
#define SMHIP_PREC_FP32 0
#define SMHIP_PREC_BF16 1

/* Quantised weight formats (values follow the reference QuantDType enum, QuantDType.cs). */
#define SMHIP_QTYPE_F32 0
#define SMHIP_QTYPE_Q8_0 8
#define SMHIP_QTYPE_Q4_K 12

typedef void* smhip_stream_t;

/* ---------------------------------------------------------------- runtime */
const char* smhip_last_error(void);
int smhip_version(void);
/* Number of visible HIP devices (0 when no GPU). */
int smhip_device_count(void);

/* ---------------------------------------------------------------- GradientMapping slots
 * (SharpMind.Core/Training/GradientMapping.cs:26-106, keys SharpMindConfig.cs:35-41) */

/* gradlinear -> GradientMapping.Linear (GradientMapping.cs:26-34, GradientKernels.cs:50-291).
 * dY [M,Out], X [M,In], W [Out,In].  dX [M,In] = dY W (overwritten, may be NULL);
 * dW [Out,In] += dY^T X (may be NULL); db [Out] += sum_rows dY (may be NULL). */
int smhip_grad_linear(const float* dY, const float* X, const float* W, float* dW, float* db,
                      float* dX, int M, int In, int Out, int precision, smhip_stream_t stream);

/* gradrmsnorm -> GradientMapping.RMSNorm (GradientMapping.cs:41-48, GradientKernels.cs:303-337).
 * xNorm [T,D] = x*rmsInv saved by forward; dw [D] += (may be NULL: frozen weight). */
int smhip_grad_rmsnorm(const float* dY, const float* xNorm, const float* rmsInv, const float* w,
                       float* dw, float* dX, int T, int D, smhip_stream_t stream);

/* gradlayernorm -> GradientMapping.LayerNorm (GradientMapping.cs:54-62, GradientKernels.cs:345-398). */
int smhip_grad_layernorm(const float* dY, const float* x, const float* w, float* dw, float* db,
                         float* dX, int T, int D, float eps, smhip_stream_t stream);

/* gradattention -> GradientMapping.Attention (GradientMapping.cs:68-77, GradientKernels.cs:408-481).
 * One head with materialised probs [S,S]; dQ/dK/dV [S,D] overwritten. */
int smhip_grad_attention(const float* dO, const float* q, const float* k, const float* v,
                         const float* probs, float* dQ, float* dK, float* dV, int S, int D,
                         float scale, smhip_stream_t stream);

/* gradembedding -> GradientMapping.Embedding (GradientMapping.cs:84-90, GradientKernels.cs:490-506).
 * dE [V,D] += scatter of dY [T,D] rows by ids [T]; deterministic (rows summed in token order). */
int smhip_grad_embedding(const float* dY, const int32_t* ids, float* dE, int T, int D, int V,
                         smhip_stream_t stream);

/* gradactivationsilu / gradactivationgelu (GradientMapping.cs:92-106, GradientKernels.cs:559-675). */
int smhip_grad_silu(const float* dY, const float* x, float* dX, int64_t n, smhip_stream_t stream);
int smhip_grad_gelu(const float* dY, const float* x, float* dX, int64_t n, smhip_stream_t stream);

/* ---------------------------------------------------------------- TrainingOps slots
 * (SharpMind.Training/TrainingOps.cs:17-33, keys SharpMindConfig.cs:32-33) */

/* adamw -> TrainingOps.AdamWUpdate (TrainingKernels.cs:19-89).  In place on data/m/v. */
int smhip_adamw_update(float* data, const float* grad, float* m, float* v, int64_t n, float beta1,
                       float beta2, float bc1, float bc2, float lr, float eps, float decay,
                       smhip_stream_t stream);
/* gradnorm -> TrainingOps.L2NormSq (TrainingKernels.cs:94-135).  *out (device float) = sum x^2,
 * accumulated in double, deterministic. */
int smhip_l2normsq(const float* data, int64_t n, float* out, smhip_stream_t stream);
/* Gradients.ClipGlobalNorm's scale step (Gradients.cs:92-116): x *= scale for n elements. */
int smhip_scale_inplace(float* x, int64_t n, float scale, smhip_stream_t stream);

/* ---------------------------------------------------------------- QuantizationOps slots
 * QuantizedMatMulFn(float* in, byte* rawW, float* out, int M, int K, int N)
 * (QuantizationOps.cs:8-9; qmatmul_f32 :466-475, qmatmul_q8_0 :204-213, qmatmul_q4k :400-409).
 * out[M,N] = in[M,K] . W^T with W rows [N][K] in the reference byte layout. */
int smhip_qmatmul(int qtype, const float* in, const void* rawW, float* out, int M, int K, int N,
                  int precision, smhip_stream_t stream);

/* Dequant-fused bf16 MFMA GEMM through a frozen quantised weight: the forward product
 * (trans_w = 0: C[M,N] = A[M,K] . deq(W)^T, W rows [N][K]) and the dX product of the backward
 * (trans_w = 1: C[M,N] = A[M,K] . deq(W), W rows [K][N]; dX = dY W with K = Out, N = In).
 * A is bf16 with row stride lda, C fp32.  The weight values are the bit-exact dequantised fp32
 * values of the reference layout (ReadQ8_0_Scalar QuantizationKernels.Q8.cs:412-433,
 * ReadQ4K_Scalar QuantizationKernels.Q4.cs:951-981), rounded once to bf16.  The reference has
 * no backward through quantised weights; this is the dX half of QuantizedMatMulFn's gradient. */
int smhip_qgemm_bf16(int qtype, int trans_w, int M, int N, int K, const void* A, int64_t lda, const void* rawW,
                     float* C, int64_t ldc, smhip_stream_t stream);
/* The adapted projection of LoRALayer.Forward (LoRALayer.cs:52-78) through a frozen quantised
 * base, in one product: C[M,N] = A . deq(W)^T (trans_w as smhip_qgemm_bf16) + alpha2 * A2 . B2^T,
 * with A2 [M][K2] bf16 (row stride lda2, the u = x A rows) and B2 the rank operand in bf16:
 * b2_mode 2 = [N][K2] k-contiguous, 3 = [K2][N] (the reference's B [rank, out]), row stride ldb2.
 * K % 64 == 0, N % 32 == 0; C fp32. */
int smhip_qgemm_bf16_lora(int qtype, int trans_w, int M, int N, int K, const void* A, int64_t lda, const void* rawW,
                          int K2, const void* A2, int64_t lda2, int b2_mode, const void* B2, int64_t ldb2,
                          float alpha2, float* C, int64_t ldc, smhip_stream_t stream);
/* Tied LM head forward and cross-entropy backward in bf16 (BackpropEngine.cs:889-907 head,
 * CrossEntropyLoss.Compute/Backward with mean over labels != -100): logits[T,V] = x[T,d] . deq(E)^T
 * (x bf16, E the Q8_0 / Q4_K embedding table [V][d] in the reference byte layout, logits fp32),
 * dlogits = (softmax - onehot) / count in bf16, *loss = mean loss (loss may be null).  When the
 * product has at least four 128x128 tiles per CU the GEMM also emits softmax row statistics and
 * the logits are read once by the cross-entropy. */
int smhip_lm_head_ce_bf16(int qtype, int T, int V, int d, const void* x, const void* rawE, const int32_t* labels,
                          float* logits, void* dlogits, float* loss, smhip_stream_t stream);

/* Bit-exact dequantisation of a reference-layout stream of n elements
 * (ReadQ8_0_Scalar QuantizationKernels.Q8.cs:412-433, ReadQ4K_Scalar QuantizationKernels.Q4.cs:951-981). */
int smhip_dequant(int qtype, const void* raw, float* out, int64_t n, smhip_stream_t stream);

/* ---------------------------------------------------------------- BackpropEngine inline math
 * (no slot in the reference; these restate loops in SharpMind.Training/Autograd/BackpropEngine.cs) */

/* SwiGLU backward (BackpropEngine.cs:623-657): dAct, gate, up [T,F] -> dFused [T,2F] = [dGate | dUp]. */
int smhip_grad_swiglu(const float* dAct, const float* gate, const float* up, float* dFused, int T,
                      int F, smhip_stream_t stream);
/* SwiGLU forward act = silu(gate)*up (ActivationKernels.cs:194-205). */
int smhip_swiglu_forward(const float* gate, const float* up, float* act, int64_t n,
                         smhip_stream_t stream);

/* RoPE tables (RoPE.cs:99-148, no scaling): host arrays cosT/sinT [maxSeq, ropeDim/2]. */
int smhip_rope_tables(float theta, int ropeDim, int maxSeq, float* cosT, float* sinT);
/* RoPE forward / backward in place on x [B,S,H,D] with device tables (RoPE.cs:168-347);
 * neox != 0 pairs (d, d+D/2), else adjacent (2i, 2i+1). */
int smhip_rope_forward(float* x, const float* cosT, const float* sinT, int B, int S, int H, int D,
                       int neox, smhip_stream_t stream);
int smhip_rope_backward(float* dx, const float* cosT, const float* sinT, int B, int S, int H, int D,
                        int neox, smhip_stream_t stream);

/* RMSNorm forward with state (NormLayer.cs:72-89, NormKernels.cs:13-60): y = x*rmsInv*w. */
int smhip_rmsnorm_forward(const float* x, const float* w, float* y, float* rmsInv, int T, int D,
                          float eps, smhip_stream_t stream);

/* Combined softmax + cross-entropy gradient (Gradients.cs:33-84) and loss
 * (CrossEntropyLoss.cs:44-104).  dLogits [T,V] overwritten (may alias logits);
 * loss (device float, may be NULL) = mean over labels != ignoreId. */
int smhip_ce_softmax_grad(const float* logits, const int32_t* labels, float* dLogits, float* loss,
                          int T, int V, int ignoreId, float smoothing, smhip_stream_t stream);

/* Causal attention forward with materialised probs (BackpropEngine.cs:237-388, exact-exp path):
 * q [B,S,Hq,D], k/v [B,S,Hkv,D] -> probs [B,Hq,S,S], out [B,S,Hq*D]. */
int smhip_attention_forward_probs(const float* q, const float* k, const float* v, float* probs,
                                  float* out, int B, int S, int Hq, int Hkv, int D,
                                  smhip_stream_t stream);

/* Causal GQA attention on bf16 MFMA without materialised probabilities (the engine's
 * bf16 path; mathematically the forward of BackpropEngine.cs:237-388 and the backward of
 * GradientKernels.cs:408-481).  Row r = b*S + s of q holds head h at columns [h*D, h*D+D)
 * (row stride ldq elements); likewise k/v with Hkv heads.  q/k/v/o/dO are bf16 (uint16
 * bits), lse [B,Hq,S] fp32 in log2 units, dq/dk/dv fp32 (overwritten).  S % 128 == 0,
 * D in {64, 128}.  Backward is deterministic (no atomics). */
int smhip_flash_attention_forward(const void* q, const void* k, const void* v, void* o, float* lse,
                                  int B, int S, int Hq, int Hkv, int D, int64_t ldq, int64_t ldk,
                                  int64_t ldv, int64_t ldo, smhip_stream_t stream);
int smhip_flash_attention_backward(const void* q, const void* k, const void* v, const void* o,
                                   const void* dO, const float* lse, float* dq, float* dk, float* dv,
                                   int B, int S, int Hq, int Hkv, int D, int64_t ldq, int64_t ldk,
                                   int64_t ldv, int64_t ldo, int64_t lddo, int64_t lddq,
                                   int64_t lddk, int64_t lddv, smhip_stream_t stream);

/* Allocation-free variant of smhip_flash_attention_backward.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments and results (bit for bit) as
 * smhip_flash_attention_backward; the scratch it needs, B*Hq*S*(2*D+1)*4 + 256 bytes, comes from a
 * fixed per-device array of smhip_flash_attention_backward_noalloc_limit() bytes (80 MiB) instead of
 * the library's workspace pool, and larger problems return SMHIP_EINVAL.  The entry calls no
 * hipMalloc/hipFree.  All calls on one device share that array: calls that overlap on one device
 * (several streams or threads at once) race and must be serialised by the caller. */
int smhip_flash_attention_backward_noalloc(const void* q, const void* k, const void* v, const void* o,
                                           const void* dO, const float* lse, float* dq, float* dk, float* dv,
                                           int B, int S, int Hq, int Hkv, int D, int64_t ldq, int64_t ldk,
                                           int64_t ldv, int64_t ldo, int64_t lddo, int64_t lddq, int64_t lddk,
                                           int64_t lddv, smhip_stream_t stream);
int smhip_flash_attention_backward_noalloc_limit(int64_t* bytes);

/* General dense GEMM on MFMA: C[M,N] = alpha * sum_k A(m,k) B(n,k) + beta * C.
 * Operand modes: 0 fp32 k-contiguous (X[r*ld + k]), 1 fp32 row-contiguous (X[k*ld + r]),
 * 2 bf16 k-contiguous, 3 bf16 row-contiguous.  C is fp32 (c_bf16 = 0) or bf16.  split_k > 1 splits
 * the reduction deterministically; split_k = 0 lets the bf16 path choose tile and split.  precision: SMHIP_PREC_FP32 (fp32 MFMA) or SMHIP_PREC_BF16. */
int smhip_gemm(int M, int N, int K, int a_mode, const void* A, int64_t lda, int b_mode, const void* B,
               int64_t ldb, float alpha, float beta, void* C, int64_t ldc, int c_bf16, int split_k,
               int precision, smhip_stream_t stream);

/* TensorQuantizer.Quantize for Q8_0 / Q4_K on the device (TensorQuantizer.cs:80-144,
 * TensorQuantizer.KQuant.cs:173-225): same bytes as the reference encoder. */
int smhip_quantize(int qtype, const float* x, int64_t n, void* out, smhip_stream_t stream);

/* ---------------------------------------------------------------- training engine
 * One resident fwd+bwd+optimizer step of a decoder (TrainLoop.ForwardBackward +
 * BackpropEngine + Gradients.ClipGlobalNorm + AdamW.Update; TrainLoop.cs:100-135,222-243).
 * Tensor names: "emb", "norm_f", "l<i>.norm1|norm2|q_norm|k_norm", full-parameter
 * "l<i>.wqkv|wo|wgu|wd" ([Out][In] fp32) and "l<i>.bqkv|bo|bgu|bd", LoRA
 * "l<i>.lora.<q|k|v|o|gate|up|down>.<A|B>" (A [In,r], B [r,Out] fp32).  In LoRA mode
 * "emb" and "l<i>.w*" take the reference's raw Q8_0 / Q4_K bytes. */
typedef struct {
  int n_layers, d_model, n_heads, n_kv_heads, head_dim, ffn_dim, vocab;
  int batch, seq;
  float norm_eps, rope_theta;
  int rope_neox, qk_norm;
  int base_qtype;       /* SMHIP_QTYPE_F32: full-parameter training; Q8_0 / Q4_K: frozen LoRA base */
  int lora_rank;
  float lora_alpha;
  int precision;        /* SMHIP_PREC_FP32 | SMHIP_PREC_BF16 */
  int use_bias;
  float lr, beta1, beta2, adam_eps, weight_decay; /* AdamW (Optimizers/AdamW.cs:22-41) */
  float max_grad_norm;  /* <= 0: no clipping (TrainConfig.GradClipNorm, TrainConfig.cs:20) */
} smhip_model_config;

int smhip_engine_create(const smhip_model_config* cfg, void** engine);
int smhip_engine_destroy(void* engine);
int smhip_engine_param_count(void* engine, int64_t* trainable, int64_t* frozen);
int smhip_engine_set_tensor(void* engine, const char* name, const void* host, int64_t nbytes);
/* which = 0: parameter, 1: gradient, 2: AdamW first moment m, 3: AdamW second moment v */
int smhip_engine_get_tensor(void* engine, const char* name, int which, void* host, int64_t nbytes);
/* Synthetic initialisation on the device: N(0,0.02) weights (quantised in LoRA mode), norms 1,
 * biases 0, LoRA A Kaiming-uniform, B ~ N(0,1e-3). */
int smhip_engine_init_synthetic(void* engine, uint64_t seed);
/* ids/labels: device int32 [batch*seq] (label -100 = ignored); loss: device float or NULL.
 * Zeroes the gradients first (optimizer.ZeroGrad at the start of a window, TrainLoop.cs:108-109),
 * then runs TrainLoop.ForwardBackward (TrainLoop.cs:222-243). */
int smhip_engine_forward_backward(void* engine, const int32_t* ids, const int32_t* labels, float* loss,
                                  smhip_stream_t stream);
/* Gradient accumulation over micro-batches (TrainLoop.RunAsync, TrainLoop.cs:104-120): with
 * accumulate != 0 the gradients of this micro-batch are ADDED to those already held (no zeroing),
 * so GradAccumSteps micro-batches followed by one optimizer step reproduce the reference loop.
 * accumulate == 0 is smhip_engine_forward_backward. */
int smhip_engine_forward_backward_accum(void* engine, const int32_t* ids, const int32_t* labels, float* loss,
                                        int accumulate, smhip_stream_t stream);
/* optimizer.ZeroGrad (Optimizers/AdamW.cs:91-94): all trainable gradients to 0 on `stream`. */
int smhip_engine_zero_grad(void* engine, smhip_stream_t stream);
/* _optimizer.LearningRate = _scheduler.GetLr(step + 1) (TrainLoop.cs:122-123): the learning rate the
 * next smhip_engine_optimizer_step uses.  Finite and >= 0. */
int smhip_engine_set_lr(void* engine, float lr);
int smhip_engine_get_lr(void* engine, float* lr);
/* Clip (if configured) + AdamW; grad_norm_sq: device float or NULL (pre-clip sum of squares). */
int smhip_engine_optimizer_step(void* engine, float* grad_norm_sq, smhip_stream_t stream);
int smhip_engine_step(void* engine, const int32_t* ids, const int32_t* labels, float* loss,
                      smhip_stream_t stream);
/* Execution mode of forward_backward (no reference counterpart: the reference runs on the
 * CPU).  on != 0: the first call records the step's ~1500 kernel launches as a HIP graph on a
 * private stream (after one eager pass that also produces that call's result), later calls copy
 * ids/labels into engine buffers and replay the graph on the caller's stream.  Results are
 * bit-identical to eager mode.  Calls made while the live profiler is active run eagerly. */
int smhip_engine_use_graph(void* engine, int on);
/* Checkpoint.Save (Checkpoint.cs:27-82) with AdamW.SaveState (Optimizers/AdamW.cs:96-105):
 * writes <dir>/model.bin, optimizer.bin (when with_optimizer) and meta.json in the reference's
 * byte format, creating dir.  The tensors are the reference's trainable parameter list (names,
 * order, [In, Out] weight layout); loss NaN and note NULL are written as JSON null. */
int smhip_engine_save_checkpoint(void* engine, const char* dir, int with_optimizer, int step, float loss,
                                 const char* note);
/* Checkpoint.Load (Checkpoint.cs:161-237) with AdamW.LoadState (Optimizers/AdamW.cs:107-117):
 * tensors matched by name (repeated names in order), unknown names skipped, an element-count
 * mismatch is an error naming the tensor.  With with_optimizer and an optimizer.bin present, m, v
 * and lr are restored and the AdamW step becomes meta.json's step.  step / loss (nullable)
 * receive meta.json's values (0 / NaN without one). */
int smhip_engine_load_checkpoint(void* engine, const char* dir, int with_optimizer, int* step, float* loss);
/* Checkpoint.FindLatest (Checkpoint.cs:117-145): path of the latest "step-*" directory under dir
 * into out (cap bytes); returns 1 if found, 0 if none. */
int smhip_checkpoint_find_latest(const char* dir, char* out, int64_t cap);
/* GgufLoader.LoadAllWeights / LoadSingleTensor (SharpMind.Model/Format/GgufLoader.cs:435-600) for a LoRA engine's frozen
 * base: token_embd, blk.<i>.attn_q|attn_k|attn_v|attn_output|ffn_gate|ffn_up|ffn_down.weight (ggml type
 * = base_qtype), the norms attn_norm, ffn_norm, attn_q_norm, attn_k_norm, output_norm (F32 or F16).
 * Names, types and shapes are checked against the engine; an untied output.weight is an error. */
int smhip_engine_load_gguf(void* engine, const char* path);
/* GGUF header inspection (GgufLoader.LoadMeta, GgufLoader.cs:124-177): the tensor table of a file.
 * dims receives 8 entries (innermost first, padded with 1); file_offset is absolute. */
int smhip_gguf_tensor_count(const char* path, int64_t* count);
int smhip_gguf_tensor_info(const char* path, int64_t index, char* name, int64_t cap, int* ggml_type, int* n_dims,
                           int64_t* dims, int64_t* file_offset);
/* Diagnostics: copy a saved activation of the last forward to host memory.  what: "h_in", "h_mid",
 * "xn1", "qkv", "q", "k", "v", "o", "gu", "act" (of `layer`), "h_fin", "logits" ("logits" holds
 * dLogits after a fp32-mode backward).  Element type is bf16 for "xn1|q|k|v|o|gu|act" (and "qkv" with
 * head_dim 64 or 128) in bf16 mode, fp32 otherwise. */
int smhip_engine_read_activation(void* engine, const char* what, int layer, void* host, int64_t nbytes);
/* Live kernel timing on the calling thread: between begin and end, the GEMM launcher times its main
 * kernel with start/end events taken by the dispatch (hipExtLaunchKernelGGL) and the flash-attention
 * launchers bracket their kernels with HIP events on the launch stream.  end synchronises and writes
 * out[3*c + {0,1,2}] = (milliseconds, launches, algorithmic flops) for category c
 * (0 = MFMA GEMM kernel, 1 = flash forward, 2 = flash backward kernels, 3 = MFMA GEMM kernel with a
 * quantised column-plane B operand, i.e. the backward dX products through the frozen base), c < ncat. */
int smhip_profile_begin(int max_events);
int smhip_profile_end(double* out, int ncat);
/* Measurement, no reference counterpart: the bf16 MFMA rate (TFLOP/s) the device sustains with register
 * operands and no memory traffic, one 8-wave workgroup per CU (about 0.1 s).  bench.py reports it
 * beside the published dense peak. */
int smhip_probe_mfma_bf16(double* tflops);
/* Uniform random token ids in [0, vocab) (synthetic batches). */
int smhip_fill_token_ids(int32_t* ids, int64_t n, uint64_t seed, int vocab, smhip_stream_t stream);

/* ---------------------------------------------------------------- host-pointer slot entries
 * Same semantics as the device entries above, on host memory (synchronous).  These are
 * what SharpMind.HIP's [PuzzlePeice] methods P/Invoke. */
int smhip_host_grad_linear(const float* dY, const float* X, const float* W, float* dW, float* db,
                           float* dX, int M, int In, int Out, int precision);
int smhip_host_grad_rmsnorm(const float* dY, const float* xNorm, const float* rmsInv,
                            const float* w, float* dw, float* dX, int T, int D);
int smhip_host_grad_layernorm(const float* dY, const float* x, const float* w, float* dw,
                              float* db, float* dX, int T, int D, float eps);
int smhip_host_grad_attention(const float* dO, const float* q, const float* k, const float* v,
                              const float* probs, float* dQ, float* dK, float* dV, int S, int D,
                              float scale);
int smhip_host_grad_embedding(const float* dY, const int32_t* ids, float* dE, int T, int D, int V);
int smhip_host_grad_silu(const float* dY, const float* x, float* dX, int64_t n);
int smhip_host_grad_gelu(const float* dY, const float* x, float* dX, int64_t n);
int smhip_host_adamw_update(float* data, const float* grad, float* m, float* v, int64_t n,
                            float beta1, float beta2, float bc1, float bc2, float lr, float eps,
                            float decay);
int smhip_host_l2normsq(const float* data, int64_t n, float* out);
int smhip_host_qmatmul(int qtype, const float* in, const void* rawW, float* out, int M, int K,
                       int N);

#ifdef __cplusplus
}
#endif
#endif
