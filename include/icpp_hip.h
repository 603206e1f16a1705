/*
 * icpp_hip.h -- C ABI of libicpp_hip.so, the gfx950 (MI355X) kernel library
 * behind the tuner's "compile / run / benchmark" steps.
 *
 * The reference binds its device code in-process through TileLang: each kernel
 * module compiles a shape-specialised prim_func and calls it on torch tensors
 * (kernel/tilelang/gemm/gemm.py:84-89, gemm_bias_act.py:91-96,
 * gemm_bias_layernorm.py:167-188, conv/conv2d.py:282-290).  Here the kernels are
 * compiled ahead of time as a fixed set of tile instances; "compile" resolves a
 * config to an instance index and "run" is one of the launchers below.
 *
 * Conventions
 *  - Plain C types only; tensors are device pointers, row-major, contiguous.
 *  - Return 0 on success, a negative ICPP_E_* code on a rejected call, or a
 *    positive hipError_t from the launch.  icpp_last_error() describes the last
 *    failure of the calling thread.
 *  - Launchers never allocate device memory: split-K partials and LayerNorm
 *    statistics live in a caller-owned workspace of icpp_workspace_bytes().
 *  - Launches are asynchronous on `stream` (a hipStream_t; NULL = default).
 *  - Stateless and reentrant; concurrent calls may share instances.
 */
#ifndef ICPP_HIP_H
#define ICPP_HIP_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ICPP_ABI_VERSION 2

/* instance families */
enum icpp_family {
  ICPP_FAMILY_GEMM = 0,        /* dense GEMM, epilogue bias/act or split-K partials */
  ICPP_FAMILY_GEMM_LN_STATS = 1,/* GEMM+bias writing X and per-(row, column block) LN statistics */
  ICPP_FAMILY_GEMM_LN_ROW = 2, /* GEMM+bias+LayerNorm with whole rows per workgroup */
  ICPP_FAMILY_CONV2D = 3,      /* NHWC x HWIO implicit-GEMM conv2d */
  ICPP_NUM_FAMILIES = 4
};

/*
 * Strategy code for the LayerNorm entry points, beside the families above (it is
 * not an instance family): `inst` is an f16 ICPP_FAMILY_GEMM instance, run with
 * the co-resident row-block epilogue (see icpp_gemm_bias_layernorm).
 */
enum { ICPP_LN_CORESIDENT = 16 };

enum icpp_dtype { ICPP_F16 = 0, ICPP_BF16 = 1, ICPP_FP8_E4M3 = 2, ICPP_F32 = 3 /* row ops only */ };
enum icpp_act { ICPP_ACT_NONE = 0, ICPP_ACT_RELU = 1, ICPP_ACT_GELU_TANH = 2, ICPP_ACT_SILU = 3,
                ICPP_ACT_GELU_ERF = 4 /* 0.5 x (1 + erf(x / sqrt 2)), torch's default F.gelu */ };

enum icpp_status {
  ICPP_OK = 0,
  ICPP_E_INSTANCE = -1,  /* bad family / instance index */
  ICPP_E_SHAPE = -2,     /* shape not supported by the instance (divisibility, alignment) */
  ICPP_E_WORKSPACE = -3, /* workspace missing or too small */
  ICPP_E_ARG = -4        /* other invalid argument */
};

typedef struct icpp_tile {
  int family;      /* enum icpp_family */
  int dtype;       /* enum icpp_dtype of A and B */
  int block_m, block_n, block_k;
  int waves_m, waves_n;
  int stages;      /* LDS buffers */
  int mfma_m, mfma_n, mfma_k;
  int lds_bytes;   /* static LDS of the mainloop kernel */
  int threads;
  char name[96];
} icpp_tile_t;

int icpp_abi_version(void);
const char* icpp_last_error(void);

/* Instance table: the tuner's candidate space (replaces get_configs(), gemm.py:24-48). */
int icpp_num_instances(int family);
int icpp_instance_info(int family, int idx, icpp_tile_t* out);

/* Bytes of workspace a call needs (0 when none). */
size_t icpp_workspace_bytes(int family, int inst, int M, int N, int K, int split_k);

/*
 * C[M,N] = act(scale_a*scale_b * A[M,K].B[K,N] + bias[N]).
 * Replaces the TileLang kernels of gemm.py:61-79 (bias = NULL, act = NONE) and
 * gemm_bias_act.py:59-86 (bias + ReLU), and adds GELU-tanh / SiLU and the fp8
 * e4m3 per-tensor-scaled variant.  Output and bias dtypes follow the instance
 * dtype: f16 -> f16 out/bias, bf16 -> bf16 out/bias, fp8 -> bf16 out, f32 bias.
 * split_k > 1 accumulates K slices in the fp32 workspace and reduces them.
 * Requires K % (block_k * split_k) == 0, N % 8 == 0, ld* % 8 == 0.
 */
int icpp_gemm(int inst, const void* A, const void* B, const void* bias, void* C,
              int M, int N, int K, int lda, int ldb, int ldc, int act,
              float scale_a, float scale_b, int split_k,
              void* workspace, size_t ws_bytes, void* stream);

/*
 * Y[M,N] = LayerNorm_N(A.B + bias) * gamma + beta, f16 in / f16 out, fp32 statistics.
 * Replaces build_fused_kernel (gemm_bias_layernorm.py:167-188: GEMM+bias kernel
 * :61-88 followed by the row LayerNorm kernel :101-162).  `family` selects the
 * strategy: ICPP_FAMILY_GEMM_LN_ROW (whole row per workgroup, N <= block_n,
 * no workspace), ICPP_FAMILY_GEMM_LN_STATS (GEMM writes X into Y plus
 * per-block (mean, M2) into the workspace, then a finalize pass normalises Y),
 * ICPP_FAMILY_GEMM (below) or ICPP_LN_CORESIDENT (below).
 * The reference keeps X in fp32 between its two kernels (:59, :66, :103); the
 * two-launch strategies here keep X in Y as f16 values centred on the mean of
 * their (row, wave column block), with that mean in fp32 in the workspace, so a
 * row offset far above the row's spread loses no precision.
 * ICPP_LN_CORESIDENT (inst: an f16 ICPP_FAMILY_GEMM instance whose tile has 2+
 * stages) keeps X in registers: the
 * workgroups of a row block exchange their (mean, M2) through the workspace and
 * normalise their tiles from registers.  Row blocks beyond what the device keeps
 * resident at once run in rounds of one launch (each XCD starts its workgroups in
 * order, and a round's row blocks are all resident before the next round's take
 * a CU), or in even chunks, one launch each, when a round does not split over the
 * 8 XCDs.  Its workspace
 * (icpp_gemm_bias_layernorm_workspace_bytes) ends in a counter block that must be
 * zero before the first call on it; every call leaves it zero.  Calls that share a
 * workspace, or that run at the same time on different streams, must not overlap.
 * ICPP_E_SHAPE when one row block cannot be resident at once (N too wide for the
 * tile) or its statistics do not fit two LDS stage arrays.
 */
int icpp_gemm_bias_layernorm(int family, int inst, const void* A, const void* B, const void* bias,
                             const void* gamma, const void* beta, void* Y,
                             int M, int N, int K, float eps,
                             void* workspace, size_t ws_bytes, void* stream);

/*
 * Y = LayerNorm_N(A[M,K] @ B[K,N] + bias + residual) * gamma + beta: the
 * attention-output and FFN-output blocks of the reference's BERT layer
 * (evaluation/end2end.py:76-79, :84-87: matmul + bias, + residual, F.layer_norm).
 * residual is [M, N] f16 (may be Y itself: each element is read before it is
 * written, by the same lane); null gives icpp_gemm_bias_layernorm.
 * family may also be ICPP_FAMILY_GEMM (an f16 GEMM instance): a GEMM + bias into
 * Y (stored centred on per-(row, wave column block) means, the means in the
 * workspace), then the row LayerNorm in place -- the same HBM traffic as the
 * two-pass family, any GEMM tile.  With that family the residual must not overlap
 * Y (ICPP_E_ARG otherwise): the GEMM writes Y before the LayerNorm reads it.
 */
int icpp_gemm_bias_residual_layernorm(int family, int inst, const void* A, const void* B, const void* bias,
                                      const void* residual, const void* gamma, const void* beta, void* Y,
                                      int M, int N, int K, float eps,
                                      void* workspace, size_t ws_bytes, void* stream);

/*
 * Workspace bytes icpp_gemm_bias_layernorm / icpp_gemm_bias_residual_layernorm need
 * for `family` (ICPP_FAMILY_GEMM_LN_ROW, _LN_STATS, ICPP_FAMILY_GEMM or
 * ICPP_LN_CORESIDENT) and instance (0 when none).  It holds what the reference keeps
 * in its fp32 X intermediate (gemm_bias_layernorm.py:175-186 allocates it per call):
 * per-(row, column block) statistics, M * ceil(N / wave tile columns) * 4 or * 8
 * bytes; for ICPP_LN_CORESIDENT M * ceil(N / block_n) * 8 bytes (16-byte aligned),
 * then 16 bytes whose first int is set to 1 if a row block's wait ran out (its
 * workgroups were not resident together: the call's output is then invalid; the
 * word stays set until the caller clears it), then the counters, 8 bytes per
 * block_m rows.
 */
size_t icpp_gemm_bias_layernorm_workspace_bytes(int family, int inst, int M, int N, int K);

/*
 * Y[N,OH,OW,F] = conv2d(X[N,H,W,C], W[KH,KW,C,F]), f16, fp32 accumulate.
 * Replaces make_conv2d_kernel / build_conv2d_kernel (conv2d.py:208-290):
 * destination-passing like the reference's kernel(X, W, Y).
 * Requires C % 8 == 0, F % 8 == 0, (KH*KW*C) % block_k == 0 and
 * split_k <= KH*KW*C / block_k; split_k > 1 needs split_k*M*F*4 workspace bytes.
 */
int icpp_conv2d_nhwc(int inst, const void* X, const void* Wt, void* Y,
                     int N, int H, int W, int C, int F, int KH, int KW,
                     int stride, int pad, int dilation, int split_k,
                     void* workspace, size_t ws_bytes, void* stream);

/* Fused conv epilogue parts (icpp_conv2d_nhwc_fused epi_flags). */
enum icpp_conv_epi {
  ICPP_CONV_EPI_BN = 1,        /* inference BatchNorm per output channel */
  ICPP_CONV_EPI_RESIDUAL = 2,  /* + residual[N,OH,OW,F] */
  ICPP_CONV_EPI_VAR_CLAMP = 4  /* clamp var at 0 before rsqrt (with BN) */
};

/*
 * Y = act(BN(conv2d(X, W)) + residual): the conv of icpp_conv2d_nhwc with a
 * fused epilogue, act in {ICPP_ACT_NONE, ICPP_ACT_RELU}. With BN the conv value
 * is rounded to f16 first, then BN(x) = (x - mean) * rsqrt(var + eps) * gamma
 * + beta in fp32 (gamma, beta, mean, var: [F] f16); the residual (f16, Y's
 * layout) is added in fp32 and the sum rounded to f16 once. Replaces the
 * reference's fused conv kernels:
 *   conv2d_relu.py:63-143      flags 0,                      ICPP_ACT_RELU
 *   conv2d_bn.py:67-156        BN (eps 1e-3 there),          ICPP_ACT_NONE
 *   conv2d_bn_relu.py:185-269  BN (eps 1e-5),                ICPP_ACT_RELU
 *   conv_bn_add_relu.py:73-166 BN|RESIDUAL|VAR_CLAMP (1e-5), ICPP_ACT_RELU
 * Same shape rules as icpp_conv2d_nhwc; epilogue pointers 16-byte aligned.
 */
int icpp_conv2d_nhwc_fused(int inst, const void* X, const void* Wt, void* Y, const void* residual,
                           const void* gamma, const void* beta, const void* mean, const void* var,
                           float eps, int epi_flags, int act,
                           int N, int H, int W, int C, int F, int KH, int KW,
                           int stride, int pad, int dilation, int split_k,
                           void* workspace, size_t ws_bytes, void* stream);

/*
 * Row operations over the last dimension of a row-major [M, N] tensor with row
 * stride ld >= N (elements); dtype ICPP_F16, ICPP_BF16 or ICPP_F32, fp32
 * arithmetic. The 16-byte path needs N, the strides and the pointers to be
 * multiples of 16 bytes; otherwise a per-element path runs. Rows up to
 * 8192 x (16 / element size) columns (16-byte path) or 16384 (per-element).
 */

/*
 * Y = (X - mean) * rstd * W + B per row, rstd = 1 / sqrt(var + eps) with the
 * centred (two-pass) variance; mean, rstd: [M] fp32 outputs (either may be
 * null). Replaces _layer_norm_fwd_fused and LayerNorm.forward
 * (kernel/triton/layernorm.py:48-91, :219-244).
 */
int icpp_layernorm_fwd(int dtype, const void* X, const void* W, const void* B, void* Y,
                       float* mean, float* rstd, int M, int N, int ldx, int ldy, float eps,
                       void* stream);

/*
 * Workspace bytes icpp_layernorm_bwd needs for these sizes (0 when N is beyond
 * the backward's limit: 16384 columns of a 16-bit type, 8192 of f32, 4096 on
 * the per-element path).
 */
size_t icpp_layernorm_bwd_workspace_bytes(int dtype, int M, int N, int ld);

/*
 * LayerNorm backward from the forward's mean / rstd: DX ([M, N], ld), DW, DB
 * ([N], W's dtype). Replaces _layer_norm_bwd_dx_fused + _layer_norm_bwd_dwdb
 * and LayerNorm.backward (layernorm.py:128-207, :246-275); dw / db are summed
 * in fp32 in a fixed order (deterministic).
 */
int icpp_layernorm_bwd(int dtype, const void* DY, const void* X, const void* W,
                       const float* mean, const float* rstd, void* DX, void* DW, void* DB,
                       int M, int N, int ld, void* workspace, size_t ws_bytes, void* stream);

/*
 * Y = softmax(X) per row (exp(x - max) / sum). Replaces softmax_kernel and
 * softmax (kernel/triton/softmax.py:32-55, :73-102).
 */
int icpp_softmax(int dtype, const void* X, void* Y, int M, int N, int ldx, int ldy, void* stream);

/*
 * Y = softmax(X * scale + mask[row % mask_rows]) per row, in one pass: the
 * attention scores of the reference's BERT layer (evaluation/end2end.py:52-66:
 * matmul(q, k^T) / sqrt(head_size) + causal mask, then softmax).  mask is
 * [mask_rows, N] in X's dtype with row stride N, or null (scale only); the
 * arithmetic is fp32.  Same shape limits as icpp_softmax.
 */
int icpp_softmax_scaled_masked(int dtype, const void* X, void* Y, const void* mask, float scale, int M, int N,
                               int ldx, int ldy, int mask_rows, void* stream);

/*
 * Attention head layout of the reference's BERT layer, head_dim 64 (f16 / bf16).
 * icpp_qkv_split_heads replaces `qkv + qkv_bias`, `chunk(3)`, transpose_for_scores
 * and the three permute(0, 2, 1, 3).contiguous() copies plus the k rearrange to
 * [(b h), d, s] (evaluation/end2end.py:48-58): QKV [batch*seq, 3*heads*64] row-major
 * (+ bias [3*heads*64], or null) -> Q [batch, heads, seq, 64] and, with layout 0,
 * K^T [batch, heads, 64, seq] in K and V [batch, heads, seq, 64]; with layout 1,
 * K [batch, heads, seq, 64] and V^T [batch, heads, 64, seq] (icpp_attention_fwd's
 * operands).  The bias add is one fp32 add rounded to the dtype.
 * icpp_merge_heads replaces the context reshape back to [batch*seq, heads*64]
 * (end2end.py:72-73): X [batch, heads, seq, 64] -> Y [batch*seq, heads*64].
 * Pointers 16-byte aligned; batch*seq*heads*3*64 below 2^31.
 */
int icpp_qkv_split_heads(int dtype, const void* QKV, const void* bias, void* Q, void* K, void* V, int batch,
                         int seq, int heads, int head_dim, int layout, void* stream);
int icpp_merge_heads(int dtype, const void* X, void* Y, int batch, int seq, int heads, int head_dim, void* stream);

/*
 * Fused attention of the reference's BERT layer (evaluation/end2end.py:59-73:
 * baddbmm(q, k) * 1/sqrt(d) + causal mask, softmax, einsum with v, reshape to
 * [b, t, h*d]): O [batch*seq, heads*64] = softmax(Q K^T * scale + mask) V per
 * (batch, head), from Q and K [batch, heads, seq, 64] and VT [batch, heads, 64, seq]
 * (icpp_qkv_split_heads layout 1).  mask is [seq, seq] in the data type, or null.
 * Scores and softmax in fp32; P is rounded to the data type before P V.
 * f16 / bf16, head_dim 64, seq a multiple of 32 up to 512.
 */
int icpp_attention_fwd(int dtype, const void* Q, const void* K, const void* VT, const void* mask, float scale, void* O,
                       int batch, int seq, int heads, int head_dim, void* stream);

/*
 * icpp_gemm without a workspace argument and without any device allocation: no
 * counterpart in the reference.  For callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, kernels and results as icpp_gemm; with
 * split_k > 1 the fp32 partials live in a static device array of
 * ICPP_NOALLOC_SCRATCH_BYTES per GPU (held until the process ends), so calls need
 * split_k * M * N * 4 <= ICPP_NOALLOC_SCRATCH_BYTES (ICPP_E_WORKSPACE otherwise).
 * Every call on one GPU shares that array: calls that overlap in time on one GPU
 * race; calls serialised on one stream are safe.
 */
#define ICPP_NOALLOC_SCRATCH_BYTES (16u << 20)
int icpp_gemm_noalloc(int inst, const void* A, const void* B, const void* bias, void* C,
                      int M, int N, int K, int lda, int ldb, int ldc, int act,
                      float scale_a, float scale_b, int split_k, void* stream);

/*
 * fp8 decode over pre-packed weights: no counterpart in the reference (which has
 * no fp8 kernel).  For callers that keep B fixed across calls (weights in serving)
 * and run M <= 32 rows at a time, where icpp_gemm needs split-K and a second launch.
 *
 * icpp_fp8_pack_b: Bp = B [K, N] (fp8 e4m3, row-major, N contiguous) rearranged
 * so that each 16-column block is one contiguous run over K: for block nb and
 * K step s (128 rows), 2 KiB at byte ((nb * K / 128 + s) * 64 + l) * 32, whose
 * 32 bytes for lane l are B[128 s + 32 (l / 16) + t][16 nb + l % 16], t = 0..31
 * (the 16x16x128 fp8 MFMA operand layout).  Bp holds K * N bytes, 16-byte aligned.
 * Needs K % 128 == 0 and N % 16 == 0.  Run once per weight matrix.
 *
 * icpp_fp8_gemm_packed: C[M,N] = act(scale_a*scale_b * A[M,K] @ B[K,N] + bias[N])
 * with B given packed; A fp8 row-major (lda = K), bias f32 or null, C bf16
 * (ldc = N): the types and epilogue of icpp_gemm's fp8 instances.  1 <= M <= 32,
 * K % 128 == 0, N % 16 == 0, 16-byte aligned pointers.  One launch, no workspace.
 */
int icpp_fp8_pack_b(const void* B, void* Bp, int K, int N, void* stream);
int icpp_fp8_gemm_packed(const void* A, const void* Bp, const void* bias, void* C, int M, int N, int K, int act,
                         float scale_a, float scale_b, void* stream);

/*
 * Measurement aid, no counterpart in the reference (whose harness reads clocks
 * from the NVIDIA profiler, motivation/exp_2/profile.py:39-53): one wave reads the
 * shader-clock counter and the 100 MHz real-time counter, sleeps until `seconds`
 * of real time have passed, and writes out[0] = shader-clock ticks, out[1] =
 * real-time ticks (device memory, 2 x uint64, 8-byte aligned).  Launched on its own
 * stream beside a kernel, out[0] / out[1] * 100 MHz is the shader clock the chip
 * held under that load.  seconds in (0, 10].
 */
int icpp_clock_probe(unsigned long long* out, double seconds, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ICPP_HIP_H */
