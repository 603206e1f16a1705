// MFMA tile kernels for gfx950 (MI355X / CDNA4).
//
// One templated mainloop serves every fused op of the tuner:
//   C[M,N] = epilogue( A[M,K] . B[K,N] )
// A is row-major (K contiguous) -- either a dense matrix or an NHWC activation
// gathered on the fly (implicit-GEMM conv); B is row-major (N contiguous), the
// layout the reference hands its kernels (gemm.py:63-65, conv2d.py:223-233 with
// the HWIO filter viewed as [KH*KW*C, F]).
//
// Data path per K tile (BK):
//   global --(buffer_load_dwordx4 ... lds: 16 B per lane straight into LDS,
//             range-checked so out-of-range lanes deliver 0)--> LDS ring of
//             STAGES buffers holding XOR-swizzled 16 B chunks
//   --> A fragments with ds_read_b128 (K contiguous per lane)
//   --> B fragments with ds_read_b64_tr_b16 / ds_read_b64_tr_b8, which transpose
//       the N-contiguous tile into the K-contiguous per-lane MFMA operand
//   --> v_mfma (16x16x32 / 32x32x16 for f16/bf16, 16x16x128 / 32x32x64 f8f6f4).
// The MFMA is issued with B as its first operand, so each lane ends up owning
// one output row and 4 consecutive output columns: epilogues store 8-byte
// (16-bit) or 16-byte (fp32) vectors and per-row reductions are lane shuffles.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

namespace icpp {

template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
// f(std::integral_constant<int, i>) for i = 0 .. N-1, unrolled at compile time
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

enum DType { DT_F16 = 0, DT_BF16 = 1, DT_FP8 = 2, DT_F32 = 3 };
enum Act { ACT_NONE = 0, ACT_RELU = 1, ACT_GELU_TANH = 2, ACT_SILU = 3, ACT_GELU_ERF = 4 };
enum Epi { EPI_STORE = 0, EPI_LN_STATS = 1, EPI_LN_ROW = 2, EPI_LN_CR = 3 };
// A operand loaders: dense rows, the NHWC implicit-GEMM gather for any C
// (per 16-byte chunk), the gather for C % BK == 0, where every K tile is one
// filter tap so the tap decomposition is per tile rather than per chunk, and the
// input halo of a 3x3 stride-1 conv tile.  A_PP, or-ed into a loader, selects the
// ping-pong mainloop (8 waves in two groups of one wave per SIMD).
enum ALoad { A_DENSE = 0, A_IM2COL = 1, A_IM2COL_TAP = 2, A_HALO = 3, A_PP = 8, A_DENSE_PP = A_DENSE | A_PP };
// LDS bytes of the input halo of a BM-row A_HALO conv tile (see gemm_kernel): the rows
// BM output pixels can span in an image of width <= 56, plus a one-row border on
// each side, 58 columns, 128 B per pixel.  Launchers check the actual width fits.
constexpr int halo_cap(int bm) { return ((bm + 55) / 56 + 3) * 58 * 128; }

typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

#define ICPP_LDS __attribute__((address_space(3)))
// kernel-local lambdas must inline: an outlined one takes its captures through scratch memory
#define ICPP_INLINE __attribute__((always_inline))
#define ICPP_BUF_DWORD3 0x00020000  // gfx9 raw buffer: 32-bit data format, no swizzle

// Fused conv epilogue (conv2d family): y = act(BN(round_f16(conv)) + residual), where
// BN(x) = (x - mean) * rsqrt(var + eps) * gamma + beta per output channel (inference
// statistics). Flags select the parts; with no flags the plain bias/act epilogue runs.
enum ConvEpiFlag { CEPI_BN = 1, CEPI_RESIDUAL = 2, CEPI_VAR_CLAMP = 4 };
struct ConvEpiArgs {
  int flags;
  float eps;
  const void* gamma;     // [N] f16
  const void* beta;      // [N] f16
  const void* mean;      // [N] f16
  const void* var;       // [N] f16; negative values clamp to 0 with CEPI_VAR_CLAMP
  const void* residual;  // [M, ldc] f16, the output's layout
};

// Division by a launch-constant divisor d >= 1 of 0 <= n < 2^31: floor(n * m / 2^p)
// with p = 31 + ceil(log2 d) and m = floor(2^p / d) + 1 < 2^32 (Granlund and
// Montgomery's round-up method: m * d - 2^p lies in [1, d] <= 2^(p - 31)).  The
// launcher computes (m, p); a division is then one 64-bit multiply and a shift
// instead of ~30 vector instructions.
struct FastDiv { uint32_t m; uint32_t p; };
__device__ __forceinline__ int fdiv(int n, FastDiv d) {
  return (int)(((uint64_t)(uint32_t)n * d.m) >> d.p);
}

// Kernel arguments (passed by value; everything the launcher resolved on the host).
struct KArgs {
  const void* A;
  const void* B;
  const void* bias;   // [N] (f16 for f16, bf16 for bf16, f32 for fp8), or null
  void* C;            // [M, ldc] output, or null when writing split-K partials
  const void* gamma;  // LN [N]
  const void* beta;   // LN [N]
  float* ws;          // split-K partials [split][M][N] f32, or LN stats [M][stat_cols][2]
  int M, N, K;
  int lda, ldb, ldc;  // in elements
  int act;
  float alpha;        // scale_a * scale_b (fp8), 1 otherwise
  float eps;
  int k_split;        // K elements per split slice (multiple of BK); the last slice may be shorter
  int splits;         // K slices (split-K); items = tiles_m * tiles_n * splits
  int tiles_m, tiles_n;
  int stat_cols;      // LN stats columns per row
  int partial;        // 1: store fp32 partials to ws[split]
  // implicit-GEMM conv geometry (A_IM2COL*); GEMM M = Nb*OH*OW, K = KH*KW*C
  int cH, cW, cC, cKH, cKW, cS, cP, cD, cOH, cOW;
  FastDiv dv_ohw, dv_ow, dv_w, dv_wp, dv_h;  // by OH*OW, OW, W, W+2, H
  uint32_t tap_rows;       // bit kh*KW set for every filter row kh (KH*KW <= 32)
  uint32_t a_bytes_total;  // X size in bytes (buffer range for the gather)
  ConvEpiArgs ce;          // fused conv epilogue (conv instances only)
  const void* residual;    // LayerNorm epilogues: [M, ldc] (output type) added before the statistics, or null
  int* ln_ctr;             // EPI_LN_CR: [tiles_m][2] arrival / departure counters (zero between calls)
  int* ln_err;             // EPI_LN_CR: set to 1 when a row block's wait ran out
  // EPI_LN_CR in rounds (0: one workgroup per tile in the usual order): each round of
  // cr_rows row blocks is split into 8 per-XCD blocks of cr_rows / cr_xa row blocks x
  // tiles_n / cr_xb tile columns
  int cr_rows, cr_xa, cr_xb;
};

template <int DT> struct DTraits;
template <> struct DTraits<DT_F16> { static constexpr int esz = 2; typedef _Float16 T; typedef _Float16 OutT; typedef _Float16 BiasT; };
template <> struct DTraits<DT_BF16> { static constexpr int esz = 2; typedef __bf16 T; typedef __bf16 OutT; typedef __bf16 BiasT; };
template <> struct DTraits<DT_FP8> { static constexpr int esz = 1; typedef uint8_t T; typedef __bf16 OutT; typedef float BiasT; };

// ---------------------------------------------------------------------------
// MFMA wrappers. Lane layouts (verified on gfx950):
//   16x16xK: operand lane l holds row/col (l%16), K slice (l/16)*EPL .. +EPL
//            result lane l holds col (l%16), rows 4*(l/16)+0..3
//   32x32xK: operand lane l holds row/col (l%32), K slice (l/32)*EPL .. +EPL
//            result lane l holds col (l%32), rows 8*(j/4)+4*(l/32)+j%4, j<16
// EPL (elements per lane) = 8 for 16-bit types, 32 for fp8.
// ---------------------------------------------------------------------------
template <int DT, int MF> struct Mfma;
template <> struct Mfma<DT_F16, 16> {
  static constexpr int KI = 32, FRAG_DW = 4, ACC = 4;
  typedef i32x4 Frag; typedef f32x4 Acc;
  static __device__ __forceinline__ Acc run(Frag a, Frag b, Acc c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};
template <> struct Mfma<DT_F16, 32> {
  static constexpr int KI = 16, FRAG_DW = 4, ACC = 16;
  typedef i32x4 Frag; typedef f32x16 Acc;
  static __device__ __forceinline__ Acc run(Frag a, Frag b, Acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};
template <> struct Mfma<DT_BF16, 16> {
  static constexpr int KI = 32, FRAG_DW = 4, ACC = 4;
  typedef i32x4 Frag; typedef f32x4 Acc;
  static __device__ __forceinline__ Acc run(Frag a, Frag b, Acc c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};
template <> struct Mfma<DT_BF16, 32> {
  static constexpr int KI = 16, FRAG_DW = 4, ACC = 16;
  typedef i32x4 Frag; typedef f32x16 Acc;
  static __device__ __forceinline__ Acc run(Frag a, Frag b, Acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};
// fp8 = OCP e4m3fn on gfx950 (format code 0 for both operands, unit E8M0 scales = 127).
template <> struct Mfma<DT_FP8, 16> {
  static constexpr int KI = 128, FRAG_DW = 8, ACC = 4;
  typedef i32x8 Frag; typedef f32x4 Acc;
  static __device__ __forceinline__ Acc run(Frag a, Frag b, Acc c) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
  }
};
template <> struct Mfma<DT_FP8, 32> {
  static constexpr int KI = 64, FRAG_DW = 8, ACC = 16;
  typedef i32x8 Frag; typedef f32x16 Acc;
  static __device__ __forceinline__ Acc run(Frag a, Frag b, Acc c) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
  }
};

// ---------------------------------------------------------------------------
// small helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, ICPP_BUF_DWORD3);
}
__device__ __forceinline__ i32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}
// 16-byte buffer load written straight to LDS (gfx950 LDS DMA): lane l of the
// wave stores to lds_wave_base + 16*l.  lds_wave_base must be wave-uniform.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, char ICPP_LDS* lds_wave_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (void ICPP_LDS*)lds_wave_base, 16, voff, soff, 0, 0);
}
// s_waitcnt vmcnt(N) leaving expcnt / lgkmcnt unconstrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
// Workgroup barrier for the LDS ring.  __syncthreads() carries a workgroup
// release fence, which must cover outstanding LDS-DMA writes and so waits for
// vmcnt(0): every barrier would drain all prefetched tiles and a deeper ring
// would buy nothing.  Here each wave has already waited (vmcnt) for its own
// loads of the tile being published, and its fragment reads of the retired
// stage were consumed by MFMAs, so a plain s_barrier suffices; the asm memory
// clobber keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
__device__ __forceinline__ void lds_store16(char ICPP_LDS* base, uint32_t off, i32x4 v) {
  *reinterpret_cast<i32x4 ICPP_LDS*>(base + off) = v;
}
// LDS fragment reads.  The restrict-qualified base gives every read alias-scope
// metadata once inlined; without it the backend cannot tell a read from the
// LDS-DMA writes still in flight into another stage, and guards it with a
// vmcnt(0) wait at basic-block boundaries -- stalling on the tile just issued.
// Ordering against LDS-DMA is the kernel's own job (per-wave vmcnt waits, then a
// workgroup barrier), which no compiler-inserted per-wave wait could provide.
__device__ __forceinline__ i32x4 lds_load16(const char ICPP_LDS* __restrict__ base, uint32_t off) {
  return *reinterpret_cast<const i32x4 ICPP_LDS*>(base + off);
}
__device__ __forceinline__ i32x2 lds_tr16(const char ICPP_LDS* __restrict__ base, uint32_t off) {
  i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((i16x4 ICPP_LDS*)(base + off));
  return __builtin_bit_cast(i32x2, v);
}
__device__ __forceinline__ i32x2 lds_tr8(const char ICPP_LDS* __restrict__ base, uint32_t off) {
  return __builtin_amdgcn_ds_read_tr8_b64_v2i32((i32x2 ICPP_LDS*)(base + off));
}

// Epilogue activations, resolved at compile time (the epilogue is instantiated
// once per activation and picked with one uniform switch per tile):
//   GELU-tanh(x) = 0.5 x (1 + tanh(u)) = x * sigmoid(2u), u = sqrt(2/pi) (x + 0.044715 x^3)
//   SiLU(x)      = x * sigmoid(x)
//   GELU-erf(x)  = 0.5 x (1 + erf(x / sqrt(2)))  (erff: the device library's, ~2 ulp)
// sigmoid(z) = 1 / (1 + exp(-z)) with the hardware exp2 and reciprocal
// (v_exp_f32, v_rcp_f32: ~1 ulp each) instead of an IEEE division; z -> -inf
// gives rcp(inf) = 0, so x * sigmoid stays finite.  GELU-tanh folds its constants
// into the exponent: exp(-2u) = 2^(x (c1 + c2 x^2)) with c1 = -2 sqrt(2/pi) log2(e)
// and c2 = 0.044715 c1 -- a multiply, an fma and a multiply ahead of the exp2
// instead of five operations (7 VALU per element with the add, reciprocal and
// final multiply, against 9).
__device__ __forceinline__ float fast_sigmoid(float z) { return __builtin_amdgcn_rcpf(1.f + __expf(-z)); }
__device__ __forceinline__ float gelu_tanh_fast(float x) {
  constexpr float C1 = -2.302208198144325f;   // -2 sqrt(2/pi) / ln 2
  constexpr float C2 = -0.1029432395800235f;  // 0.044715 * C1
  return x * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(x * fmaf(x * x, C2, C1)));
}
template <int ACT>
__device__ __forceinline__ float act_fn(float x) {
  if constexpr (ACT == ACT_RELU) return fmaxf(x, 0.f);
  else if constexpr (ACT == ACT_GELU_TANH) return gelu_tanh_fast(x);
  else if constexpr (ACT == ACT_SILU) return x * fast_sigmoid(x);
  else if constexpr (ACT == ACT_GELU_ERF) return 0.5f * x * (1.f + erff(x * 0.70710678118654752f));
  else return x;
}
// f(std::integral_constant<int, act>) for the runtime activation code act
template <typename F>
__device__ __forceinline__ void dispatch_act(int act, F&& f) {
  switch (act) {
    case ACT_RELU: f(std::integral_constant<int, ACT_RELU>{}); break;
    case ACT_GELU_TANH: f(std::integral_constant<int, ACT_GELU_TANH>{}); break;
    case ACT_SILU: f(std::integral_constant<int, ACT_SILU>{}); break;
    case ACT_GELU_ERF: f(std::integral_constant<int, ACT_GELU_ERF>{}); break;
    default: f(std::integral_constant<int, ACT_NONE>{}); break;
  }
}
// Runtime activation of the fused conv epilogue: ReLU or none (the reference's variants)
template <typename F>
__device__ __forceinline__ void dispatch_relu(int act, F&& f) {
  if (act == ACT_RELU) f(std::integral_constant<int, ACT_RELU>{});
  else f(std::integral_constant<int, ACT_NONE>{});
}
// 16-byte buffer store; offsets >= the descriptor's range are dropped by the hardware.
// Output tiles are stored with device scope (cache policy SC1: written through the
// XCD's L2), so no dirty output sits in L2 when the kernel ends: the release at the
// kernel boundary otherwise writes it all back before the next launch can start
// (2.3-2.6 us between back-to-back 56x56x64 convs against ~1.0 us written through).
constexpr int ICPP_STORE_CPOL = 16;  // SC1
__device__ __forceinline__ void buf_store16(__amdgpu_buffer_rsrc_t r, uint32_t off, i32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, ICPP_STORE_CPOL);
}
#define ICPP_OOB_OFFSET 0x80000000u  // past every store descriptor (ranges are < 2 GiB)

template <typename T> __device__ __forceinline__ float to_f32(T v) { return (float)v; }
template <typename T> __device__ __forceinline__ T from_f32(float v) { return (T)v; }

template <typename T> struct Vec4Store;
template <> struct Vec4Store<_Float16> {
  static __device__ __forceinline__ void st(void* p, f32x4 v) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    h4 h = {(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
    *reinterpret_cast<h4*>(p) = h;
  }
  static __device__ __forceinline__ void st_lds(char ICPP_LDS* p, f32x4 v) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    h4 h = {(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
    *reinterpret_cast<h4 ICPP_LDS*>(p) = h;
  }
  static __device__ __forceinline__ f32x4 ld(const void* p) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    h4 h = *reinterpret_cast<const h4*>(p);
    return f32x4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
  }
  static __device__ __forceinline__ f32x4 ld_lds(const char ICPP_LDS* p) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    h4 h = *reinterpret_cast<const h4 ICPP_LDS*>(p);
    return f32x4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
  }
};
template <> struct Vec4Store<__bf16> {
  static __device__ __forceinline__ void st(void* p, f32x4 v) {
    typedef __bf16 b4 __attribute__((ext_vector_type(4)));
    b4 h = {(__bf16)v[0], (__bf16)v[1], (__bf16)v[2], (__bf16)v[3]};
    *reinterpret_cast<b4*>(p) = h;
  }
  static __device__ __forceinline__ void st_lds(char ICPP_LDS* p, f32x4 v) {
    typedef __bf16 b4 __attribute__((ext_vector_type(4)));
    b4 h = {(__bf16)v[0], (__bf16)v[1], (__bf16)v[2], (__bf16)v[3]};
    *reinterpret_cast<b4 ICPP_LDS*>(p) = h;
  }
  static __device__ __forceinline__ f32x4 ld(const void* p) {
    typedef __bf16 b4 __attribute__((ext_vector_type(4)));
    b4 h = *reinterpret_cast<const b4*>(p);
    return f32x4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
  }
  static __device__ __forceinline__ f32x4 ld_lds(const char ICPP_LDS* p) {
    typedef __bf16 b4 __attribute__((ext_vector_type(4)));
    b4 h = *reinterpret_cast<const b4 ICPP_LDS*>(p);
    return f32x4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
  }
};
template <> struct Vec4Store<float> {
  static __device__ __forceinline__ void st(void* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; }
  static __device__ __forceinline__ void st_lds(char ICPP_LDS* p, f32x4 v) { *reinterpret_cast<f32x4 ICPP_LDS*>(p) = v; }
  static __device__ __forceinline__ f32x4 ld(const void* p) { return *reinterpret_cast<const f32x4*>(p); }
  static __device__ __forceinline__ f32x4 ld_lds(const char ICPP_LDS* p) { return *reinterpret_cast<const f32x4 ICPP_LDS*>(p); }
};

// Four consecutive elements of a vector through a range-checked buffer descriptor:
// past the range the hardware returns zeros, so the loads of an epilogue need no
// branch around them and all go out before one wait (a branch per load makes the
// compiler wait for each one in turn).  vec_rsrc covers len elements, or none for a
// null vector.  Rows are padded so that a group of 4 never straddles the end (N % 8
// == 0).  The raw result is reinterpreted as a whole vector.
template <typename T>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t vec_rsrc(const void* p, int len) {
  return make_rsrc(p, p ? (uint32_t)len * (uint32_t)sizeof(T) : 0u);
}
template <typename T> struct Vec4Ld;
template <> struct Vec4Ld<_Float16> {
  static __device__ __forceinline__ f32x4 at(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    const h4 h = __builtin_bit_cast(h4, __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, 0));
    return f32x4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
  }
  static __device__ __forceinline__ f32x4 ld(__amdgpu_buffer_rsrc_t r, int n) { return at(r, (uint32_t)n * 2u); }
};
template <> struct Vec4Ld<__bf16> {
  static __device__ __forceinline__ f32x4 at(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    typedef __bf16 b4 __attribute__((ext_vector_type(4)));
    const b4 h = __builtin_bit_cast(b4, __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, 0));
    return f32x4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
  }
  static __device__ __forceinline__ f32x4 ld(__amdgpu_buffer_rsrc_t r, int n) { return at(r, (uint32_t)n * 2u); }
};
template <> struct Vec4Ld<float> {
  static __device__ __forceinline__ f32x4 at(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
  }
  static __device__ __forceinline__ f32x4 ld(__amdgpu_buffer_rsrc_t r, int n) { return at(r, (uint32_t)n * 4u); }
};

// Per-channel BN of columns n..n+3 for the fused conv epilogue, folded to
// y = x * sc + sh with sc = rsqrt(var + eps) * gamma and sh = beta - mean * sc
// (identity without CEPI_BN or past the last column). rsqrt is v_rsq_f32 (~1 ulp);
// the fold differs from (x - mean) * rsqrt * gamma + beta by fp32 rounding only.
template <typename PT>
__device__ __forceinline__ void conv_bn4(const ConvEpiArgs& ce, int N, int n, f32x4& sc, f32x4& sh) {
  sc = f32x4{1.f, 1.f, 1.f, 1.f};
  sh = f32x4{0.f, 0.f, 0.f, 0.f};
  if (!(ce.flags & CEPI_BN) || n >= N) return;
  const f32x4 g = Vec4Store<PT>::ld((const PT*)ce.gamma + n);
  const f32x4 b = Vec4Store<PT>::ld((const PT*)ce.beta + n);
  const f32x4 m = Vec4Store<PT>::ld((const PT*)ce.mean + n);
  const f32x4 v = Vec4Store<PT>::ld((const PT*)ce.var + n);
  const bool clamp = (ce.flags & CEPI_VAR_CLAMP) != 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    sc[e] = rsqrtf((clamp ? fmaxf(v[e], 0.f) : v[e]) + ce.eps) * g[e];
    sh[e] = fmaf(-m[e], sc[e], b[e]);
  }
}
// One group of 4 outputs: round the conv value to the output type (the reference
// epilogues read it back from an f16 tile), BN, + residual, act.
template <int ACT, typename OutT>
__device__ __forceinline__ f32x4 conv_epi4(f32x4 v, f32x4 sc, f32x4 sh, f32x4 r) {
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = act_fn<ACT>(fmaf((float)(OutT)v[e], sc[e], sh[e]) + r[e]);
  return v;
}

// ---------------------------------------------------------------------------
// Tile geometry
// ---------------------------------------------------------------------------
template <int DT, int BM_, int BN_, int BK_, int WM_, int WN_, int MF_, int STAGES_>
struct Tile {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_, MF = MF_, STAGES = STAGES_;
  static constexpr int ESZ = DTraits<DT>::esz;
  static constexpr int THREADS = WM * WN * 64;
  static constexpr int WTM = BM / WM, WTN = BN / WN;  // wave tile
  static constexpr int TM = WTM / MF, TN = WTN / MF;  // MFMA tiles per wave
  typedef Mfma<DT, MF> Op;
  static constexpr int KI = Op::KI;
  static constexpr int CH = 16 / ESZ;                 // elements per 16-byte chunk
  static constexpr int ROWB_A = BK * ESZ;             // LDS bytes per A row
  static constexpr int ROWB_B = BN * ESZ;             // LDS bytes per B row
  static constexpr int CPR_A = ROWB_A / 16, CPR_B = ROWB_B / 16;
  static constexpr int A_CHUNKS = BM * CPR_A, B_CHUNKS = BK * CPR_B;
  static constexpr int SA = (A_CHUNKS + THREADS - 1) / THREADS;  // chunks per thread
  static constexpr int SB = (B_CHUNKS + THREADS - 1) / THREADS;
  static constexpr bool A_EVEN = (A_CHUNKS % THREADS) == 0, B_EVEN = (B_CHUNKS % THREADS) == 0;
  static constexpr int A_BYTES = BM * ROWB_A, B_BYTES = BK * ROWB_B;
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr int LDS_BYTES = STAGE_BYTES * STAGES;
  // LDS bank geometry (gfx950) of a ds_read_b128, as fitted to SQ_LDS_BANK_CONFLICT
  // over nine fragment-read patterns (16-bit and fp8, 16x16 and 32x32 MFMA, three
  // swizzles): 64 banks x 4 B (a 256-byte window), served 16 lanes at a time, a group
  // being the lanes that differ only in lane-id bits 0, 1, 3 and 5 ({0-3, 8-11, 32-35,
  // 40-43} and its translates) -- not 16 consecutive lanes.  A ds_read_b64_tr_b{16,8}
  // serves 32 lanes x 8 bytes.  The swizzles below make each such group touch 256
  // distinct bytes.
  static constexpr int A_SWZ_PERIOD = 16;  // rows after which a_swz repeats

  static_assert(WTM % MF == 0 && WTN % MF == 0, "wave tile must be a multiple of the MFMA tile");
  static_assert(BK % KI == 0, "BK must be a multiple of the MFMA K");
  static_assert(CPR_B >= 8, "B rows must span >= 8 chunks (128 B) for the transpose-read swizzle");
  static_assert(LDS_BYTES <= 160 * 1024, "LDS overflow");

  static_assert(A_CHUNKS % 64 == 0 && B_CHUNKS % 64 == 0, "tile loads must cover whole waves");
  static_assert((SA + SB) * (STAGES - 1) < 64, "vmcnt range");

  // A: XOR applied to the 16-byte chunk index of row r.  A 16x16 fragment read takes
  // row lane % 16 and one 16-byte chunk per 16-lane K group; under the bank model above
  // the XOR swizzles linear in the row bits (searched over all matrices on row bits
  // 0-4) for which every such read of 16-bit and fp8 data touches distinct banks in
  // each group are these (SQ_LDS_BANK_CONFLICT 0-4% on the 16x16 fp8 tiles against
  // 33-40% for the 32x32 pattern, 1-3% on the 16-bit ones).  32x32 fragment reads
  // (row lane % 32, one chunk per 32 lanes) keep the pattern that spreads 16 rows of a
  // 256-byte window over distinct chunk slots (2-6% measured; the 16x16 swizzles give
  // them 40%).  Rows of 512 bytes or more hold one row per window and use r mod 16.
  static_assert(ROWB_A >= 64, "A rows must span >= 64 bytes");
  static __device__ __forceinline__ int a_swz(int r) {
    if constexpr (MF == 32) {
      constexpr int RPB = (ROWB_A >= 256) ? 1 : (256 / ROWB_A);  // rows per 256-byte window
      constexpr int SWZ = (CPR_A < 16) ? CPR_A : 16;
      return (r / RPB) % SWZ;
    } else if constexpr (ROWB_A == 64) {
      return ((r >> 3) & 1) * 3;
    } else if constexpr (ROWB_A == 128) {
      return (((r >> 1) & 1) * 3) ^ (((r >> 3) & 1) * 5);
    } else if constexpr (ROWB_A == 256) {
      return ((r & 1) * 3) ^ (((r >> 1) & 1) * 5) ^ (((r >> 3) & 1) * 8);
    } else {
      return r & 15;
    }
  }
  static __device__ __forceinline__ uint32_t a_off(int r, int c) {
    return (uint32_t)(r * ROWB_A + ((c ^ a_swz(r)) << 4));
  }
  // B: XOR applied to the 16-byte chunk index of row k.  A transpose read
  // covers 4 rows (b16) / 8 rows (b8) per 16 lanes; the second 16 lanes of the
  // cycle either read the same rows at the next 16 columns (32x32 MFMA) or rows
  // +8 (b16, 16x16) / +32 (b8, 16x16).  The chosen bits of k separate all of
  // them into distinct bank slots; only bits that are constant per lane over
  // the K steps are used, so addresses stay base + immediate.
  // Rows of 256·n bytes take the wide pattern; other lengths (128 B, or 384 B for
  // 192-column f16 tiles, which repeat the 128-B bank pattern since 384 = 128 mod
  // 256) the narrow one, whose XOR stays inside each group of 8 chunks.
  static __device__ __forceinline__ int b_swz(int k) {
    constexpr bool WIDE = ROWB_B % 256 == 0;
    if constexpr (ESZ == 2) {
      if constexpr (MF == 16)
        return WIDE ? (((k & 3) << 1) | (((k >> 3) & 1) << 3)) : ((((k >> 1) & 1) << 1) | (((k >> 3) & 1) << 2));
      else
        return WIDE ? ((k & 3) << 2) : (((k >> 1) & 1) << 2);
    } else {
      if constexpr (MF == 16)
        return WIDE ? ((k & 7) | (((k >> 5) & 1) << 3)) : (((k >> 1) & 3) | (((k >> 5) & 1) << 2));
      else
        return WIDE ? ((k & 7) << 1) : (((k >> 1) & 3) << 1);
    }
  }
  // rows after which b_swz repeats
  static constexpr int B_SWZ_PERIOD = (ESZ == 1 && MF == 16) ? 64 : 16;
  // B: row k, logical chunk c -> byte offset in the B region. The XOR keeps the
  // rows that one transpose read touches together in distinct bank groups
  // (4 rows x 32 B for b16, 8 rows x 16 B for b8).
  static __device__ __forceinline__ uint32_t b_off(int k, int c) {
    return (uint32_t)(k * ROWB_B + ((c ^ b_swz(k)) << 4));
  }
};

// One split-K output group: C[m, n..n+3] = epilogue(sum_z ws[z][m][n..n+3]), the
// partials summed in slice order.  With ce.flags set (conv instances) the fused
// conv epilogue replaces bias/alpha.
template <int DT>
__device__ __forceinline__ void splitk_group(const float* ws, void* C, const void* bias, int M, int N, int ldc,
                                             int splits, float alpha, int act, const ConvEpiArgs& ce, int m, int n) {
  typedef typename DTraits<DT>::OutT OutT;
  typedef typename DTraits<DT>::BiasT BiasT;
  // All of a group's partial loads go out before the first add (8 at a time), so the
  // slices cost one memory round trip instead of one each; the sum stays in slice order.
  f32x4 s = {0.f, 0.f, 0.f, 0.f};
  const size_t zstride = (size_t)M * N;
  const float* w = ws + (size_t)m * N + n;
  for (int z0 = 0; z0 < splits; z0 += 8) {
    f32x4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (z0 + u < splits) v[u] = Vec4Store<float>::ld(w + (size_t)(z0 + u) * zstride);
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (z0 + u < splits) s += v[u];
  }
  if (ce.flags != 0) {
    f32x4 sc, sh;
    conv_bn4<BiasT>(ce, N, n, sc, sh);
    f32x4 r = {0.f, 0.f, 0.f, 0.f};
    if (ce.flags & CEPI_RESIDUAL) r = Vec4Store<OutT>::ld((const OutT*)ce.residual + (size_t)m * ldc + n);
    dispatch_relu(act, [&](auto ACT) { s = conv_epi4<decltype(ACT)::value, OutT>(s, sc, sh, r); });
  } else {
    f32x4 bv = {0.f, 0.f, 0.f, 0.f};
    if (bias != nullptr) bv = Vec4Store<BiasT>::ld((const BiasT*)bias + n);
    dispatch_act(act, [&](auto ACT) {
#pragma unroll
      for (int e = 0; e < 4; ++e) s[e] = act_fn<decltype(ACT)::value>(s[e] * alpha + bv[e]);
    });
  }
  Vec4Store<OutT>::st((OutT*)C + (size_t)m * ldc + n, s);
}

// ---------------------------------------------------------------------------
// The mainloop + epilogue kernel
// ---------------------------------------------------------------------------
// The A_HALO input halo: an LDS array in the kernels that use it, none in the others.
template <bool ON, int N>
struct HaloLds {
  static __device__ __forceinline__ char ICPP_LDS* ptr() {
    __shared__ __attribute__((aligned(16))) char halo[N];
    return (char ICPP_LDS*)halo;
  }
};
template <int N>
struct HaloLds<false, N> {
  static __device__ __forceinline__ char ICPP_LDS* ptr() { return nullptr; }
};

// Stage arrays 4..7 of the deeper rings, likewise present only in the kernels that use
// them (each index its own object).
template <bool ON, int N, int I>
struct ExtraStage {
  static __device__ __forceinline__ char ICPP_LDS* ptr() {
    __shared__ __attribute__((aligned(16))) char stage[N];
    return (char ICPP_LDS*)stage;
  }
};
template <int N, int I>
struct ExtraStage<false, N, I> {
  static __device__ __forceinline__ char ICPP_LDS* ptr() { return nullptr; }
};

template <int DT, int BM, int BN, int BK, int WM, int WN, int MF, int STAGES, int EPI, int ALOAD>
__global__ void __launch_bounds__(WM * WN * 64)
gemm_kernel(KArgs p) {
  typedef Tile<DT, BM, BN, BK, WM, WN, MF, STAGES> G;
  typedef typename G::Op Op;
  typedef typename Op::Frag Frag;
  typedef typename Op::Acc Acc;
  typedef typename DTraits<DT>::OutT OutT;
  typedef typename DTraits<DT>::BiasT BiasT;
  constexpr int ESZ = G::ESZ;

  // One LDS array per pipeline stage: distinct objects let the compiler see that
  // the DMA writes into one stage never alias the fragment reads of another, so
  // it does not serialise them with a vmcnt(0) wait.
  // A_HALO (3x3 stride-1 conv, C == BK): the A operand is read from one input
  // halo per tile -- the tile's output rows plus a one-pixel border, all C
  // channels -- loaded once before the mainloop; the K tiles are the 9 filter
  // taps, so the pipeline stages hold B only.
  constexpr int LOADER = ALOAD & 7;
  constexpr bool HALO = LOADER == A_HALO;
  constexpr bool DENSE = LOADER == A_DENSE;
  // A_PP: the ping-pong mainloop (two wave groups alternate between an MFMA phase
  // and a memory phase)
  constexpr bool PP = (ALOAD & A_PP) != 0;
  constexpr int HALO_CAP = halo_cap(BM);
  constexpr int SBYTES = HALO ? G::B_BYTES : G::STAGE_BYTES;  // bytes per stage array
  constexpr int A_OFF = HALO ? 0 : G::A_BYTES;                // B region offset in a stage
  constexpr int LA = HALO ? 0 : G::SA;                        // A loads per thread per tile
  __shared__ __attribute__((aligned(16))) char lds0[SBYTES];
  __shared__ __attribute__((aligned(16))) char lds1[STAGES > 1 ? SBYTES : 16];
  __shared__ __attribute__((aligned(16))) char lds2[STAGES > 2 ? SBYTES : 16];
  __shared__ __attribute__((aligned(16))) char lds3[STAGES > 3 ? SBYTES : 16];
  // the halo array exists only in A_HALO kernels, so four 40 KiB stages fill the 160 KiB exactly
  char ICPP_LDS* const halo_lds = HaloLds<HALO, HALO_CAP>::ptr();
  static_assert(!HALO || (G::ESZ == 2 && BK == 64), "A_HALO: 16-bit data, one 64-channel chunk per pixel");
  static_assert(!HALO || SBYTES * STAGES + HALO_CAP <= 160 * 1024, "A_HALO: LDS overflow");
  static_assert(STAGES >= 1 && STAGES <= 8, "1 to 8 pipeline stages");
  auto stage_base = [&](auto S) -> char ICPP_LDS* ICPP_INLINE {
    constexpr int s = decltype(S)::value;
    if constexpr (s == 0) return (char ICPP_LDS*)lds0;
    else if constexpr (s == 1) return (char ICPP_LDS*)lds1;
    else if constexpr (s == 2) return (char ICPP_LDS*)lds2;
    else if constexpr (s == 3) return (char ICPP_LDS*)lds3;
    else return ExtraStage<(STAGES > s), SBYTES, s>::ptr();
  };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  // ---- work item ----
  // An item is one output tile of one K split; a launch has one workgroup per
  // item.  The grid is remapped so each XCD takes a contiguous range of slots;
  // items are ordered split-major, then in groups of 8 tile rows (grouped-M)
  // so neighbouring slots share B panels in L2.
  struct Item { int row0, col0, kz; };
  const int tiles = p.tiles_m * p.tiles_n;
  const int nb = gridDim.x;
  int slot = blockIdx.x;
  if ((nb & 7) == 0) slot = (slot & 7) * (nb >> 3) + (slot >> 3);
  auto item_of = [&](int it) ICPP_INLINE {
    const int kz = it / tiles;
    const int t = it - kz * tiles;
    constexpr int GROUP = 8;
    const int group_size = GROUP * p.tiles_n;
    const int first_m = (t / group_size) * GROUP;
    const int gm = min(p.tiles_m - first_m, GROUP);
    return Item{(first_m + (t % group_size) % gm) * BM, ((t % group_size) / gm) * BN, kz};
  };
  // EPI_LN_CR with more row blocks than the device holds at once runs in rounds, each a
  // set of whole row blocks that fits the device.  Workgroup b runs on XCD b % 8, and
  // each XCD starts its workgroups in order, so XCD x's k-th workgroup belongs to round
  // k / (its share of a round): a round's row blocks are all resident before any
  // workgroup of the next one takes a CU, and none of their waits depends on a later
  // round.  Within a round, XCD x takes block (x / cr_xb, x % cr_xb) of the round's
  // row blocks x tile columns, so its L2 holds as few A and B panels as the usual order.
  auto cr_item = [&]() ICPP_INLINE {
    const int x = blockIdx.x & 7, k = blockIdx.x >> 3;
    const int rx = p.cr_rows / p.cr_xa, cx = p.tiles_n / p.cr_xb;
    const int r = k / (rx * cx), pp = k % (rx * cx);
    const int rb = r * p.cr_rows + (x / p.cr_xb) * rx + pp % rx;
    const int tc = (x % p.cr_xb) * cx + pp / rx;
    return Item{rb * BM, tc * BN, 0};
  };
  const Item first = (EPI == EPI_LN_CR && p.cr_rows > 0) ? cr_item() : item_of(slot);
  // a last round with fewer row blocks than a full one: its spare workgroups have no tile
  if (EPI == EPI_LN_CR && first.row0 >= p.M) return;
  const int nk = min(p.k_split, p.K - first.kz * p.k_split) / BK;  // K tiles of the item (>= 1)

  // ---- global -> LDS: buffer_load_dwordx4 ... lds (16 B per lane, range-checked:
  // out-of-range lanes deliver zeros).  Load i of wave w writes LDS chunks
  // q = i*THREADS + w*64 + lane; each lane fetches the logical chunk that the
  // XOR swizzle places in that slot, so the LDS image is the swizzled tile.
  // When THREADS is a multiple of the chunks per row (and of the swizzle
  // period), load i only moves the lane down by a fixed number of rows, so the
  // per-load part of the address is a wave-uniform scalar (soffset) and one
  // VGPR per operand suffices.
  const char* Ab = (const char*)p.A;
  const char* Bb = (const char*)p.B;
  __amdgpu_buffer_rsrc_t ra, rb;
  constexpr bool A_UNIFORM = DENSE && (G::THREADS % G::CPR_A == 0) &&
                             ((G::THREADS / G::CPR_A) % G::A_SWZ_PERIOD == 0);
  // Conv tiles keep one VGPR offset per B load (B tiles are small there), so a tile's
  // B loads share one scalar offset: no per-load scalar add in the issue-bound loop.
  constexpr bool B_UNIFORM = DENSE && (G::THREADS % G::CPR_B == 0) && ((G::THREADS / G::CPR_B) % G::B_SWZ_PERIOD == 0);
  constexpr int NA = A_UNIFORM ? 1 : G::SA;
  constexpr int NB = B_UNIFORM ? 1 : G::SB;
  constexpr bool GATHER = LOADER == A_IM2COL, TAPS = LOADER == A_IM2COL_TAP;
  uint32_t a_goff[NA];  // per-lane A byte offset within the item's rows, K offset excluded
  // general gather: chunk column, image (-1 past M) and the (0, 0)-tap input coordinates
  int a_lc[GATHER ? G::SA : 1], a_img[GATHER ? G::SA : 1], a_ih0[GATHER ? G::SA : 1], a_iw0[GATHER ? G::SA : 1];
  // per-tile-tap gather: byte offset of the chunk at tap (0, 0) (may be negative
  // at the padding border) and the set of taps that land inside the image
  int a_tbase[TAPS ? G::SA : 1];
  uint32_t a_tmask[TAPS ? G::SA : 1];  // bit t: tap t lands inside the image (KH * KW <= 32)
  // Point the loaders at item it: buffer descriptors at its rows / columns and,
  // for the conv gathers, each lane's input coordinates for its output row.
  auto setup_issue = [&](const Item& it) ICPP_INLINE {
    const int row0 = it.row0, col0 = it.col0;
    if constexpr (DENSE) {
      const uint64_t rem = (uint64_t)(p.M > row0 ? p.M - row0 : 0) * (uint64_t)p.lda * ESZ;
      ra = make_rsrc(Ab + (size_t)row0 * p.lda * ESZ, rem > 0xFFFFFFF0ull ? 0xFFFFFFF0u : (uint32_t)rem);
    } else {
      ra = make_rsrc(Ab, (uint32_t)p.a_bytes_total);
    }
    {
      const uint64_t rem = ((uint64_t)(p.K - 1) * p.ldb + (uint64_t)(p.N - col0)) * ESZ;
      rb = make_rsrc(Bb + (size_t)col0 * ESZ, rem > 0xFFFFFFF0ull ? 0xFFFFFFF0u : (uint32_t)rem);
    }
#pragma unroll
  for (int i = 0; i < (HALO ? 0 : NA); ++i) {
    const int q = tid + i * G::THREADS;
    const int r = q / G::CPR_A;
    const int c = (q % G::CPR_A) ^ G::a_swz(r);
    if constexpr (DENSE) {
      a_goff[i] = (uint32_t)(r * p.lda * ESZ + c * G::CH * ESZ);
    } else {
      const int m = row0 + r;
      const int img = fdiv(m, p.dv_ohw);
      const int rem = m - img * p.cOH * p.cOW;
      const int oh = fdiv(rem, p.dv_ow), ow = rem - oh * p.cOW;
      const int ih0 = oh * p.cS - p.cP, iw0 = ow * p.cS - p.cP;
      if constexpr (GATHER) {
        a_lc[i] = c;
        a_img[i] = (m < p.M) ? img : -1;
        a_ih0[i] = ih0;
        a_iw0[i] = iw0;
      } else {
        a_tbase[i] = (((img * p.cH + ih0) * p.cW + iw0) * p.cC + c * G::CH) * ESZ;
        uint32_t mk = 0;
        if (m < p.M) {
          if (p.cD == 1) {
            // the taps with 0 <= ih0 + kh < H and 0 <= iw0 + kw < W form a rectangle of the
            // KH x KW grid: columns kw_lo..kw_hi replicated over rows kh_lo..kh_hi
            const int kh_lo = max(0, -ih0), kh_hi = min(p.cKH - 1, p.cH - 1 - ih0);
            const int kw_lo = max(0, -iw0), kw_hi = min(p.cKW - 1, p.cW - 1 - iw0);
            if (kh_lo <= kh_hi && kw_lo <= kw_hi) {
              const uint32_t cols = ((2u << kw_hi) - 1u) & ~((1u << kw_lo) - 1u);
              const uint32_t rows = ((2u << ((kh_hi + 1) * p.cKW - 1)) - 1u) & ~((1u << (kh_lo * p.cKW)) - 1u);
              mk = cols * (p.tap_rows & rows);
            }
          } else {
            for (int tap = 0, kh = 0, kw = 0; tap < p.cKH * p.cKW; ++tap) {
              const int ih = ih0 + kh * p.cD, iw = iw0 + kw * p.cD;
              if ((unsigned)ih < (unsigned)p.cH && (unsigned)iw < (unsigned)p.cW) mk |= 1u << tap;
              if (++kw == p.cKW) { kw = 0; ++kh; }
            }
          }
        }
        a_tmask[i] = mk;
      }
      a_goff[i] = 0;
    }
  }
  };
  setup_issue(first);
  uint32_t b_goff[NB];  // per-lane B byte offset within the item's columns, K offset excluded
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int q = tid + i * G::THREADS;
    const int k = q / G::CPR_B;
    const int c = (q % G::CPR_B) ^ G::b_swz(k);
    b_goff[i] = (uint32_t)(k * p.ldb * ESZ + c * 16);
  }
  // byte offset of this wave's lane 0 within one load (wave-uniform -> SGPR)
  const int wave_slot = __builtin_amdgcn_readfirstlane(tid >> 6) * 64 * 16;
  // ---- A_HALO: the tile's input halo in LDS ----------------------------------
  // Output pixel m = (g, ow) with g = m / W the output row over all images
  // (stride 1, pad 1, 3x3: OH = H, OW = W).  The tile's rows g0 .. gl need input
  // rows g0-1 .. gl+1 of the images stacked on top of each other, 64 channels =
  // eight 16-byte chunks per pixel: halo pixel q = (row - (g0 - 1)) * W + column,
  // then one zero pixel Z after the last row.  A tap (kh, kw) of output pixel
  // (g, ow) reads halo pixel (g - g0 + kh) * W + ow + kw - 1, or Z when its input
  // column or row lies outside the image.  Without zero border columns, consecutive
  // output pixels read consecutive halo pixels also across image rows, so the
  // chunk swizzle c ^ (swz(q) & 7) keeps its pattern where an MFMA row band
  // straddles an image row (with the border columns of an earlier layout, the
  // pixel index jumped by 3 there: 24.6% and 39.2% LDS bank conflicts on the
  // 256 x 64 (32x32 MFMA) and 224 x 64 (16x16) tiles at 56 x 56 x 64).  swz(q) is
  // q >> 1 for 32x32 fragment reads and q for 16x16 ones, the best of 20 swizzles
  // measured with the conflict counters on both tiles: 17.0% and 18.0% (q >> 1 on
  // the 16x16 tile: 37.8%).  The K tiles are the 9 taps.
  constexpr int HL = HALO ? (HALO_CAP / 16 + G::THREADS - 1) / G::THREADS : 1;  // halo loads per thread
  int h_q[HALO ? G::TM : 1];       // halo pixel of this lane's row of MFMA tile tm at tap (0, 0)
  int h_vmask[HALO ? G::TM : 1];   // bit kh * 3 + kw: tap (kh, kw) reads inside the image
  int h_z = 0;                     // the zero pixel Z
  auto halo_swz = [&](int q) ICPP_INLINE { return (MF == 16 ? q : q >> 1) & 7; };
  // the halo rows of item it: first output row g0 and the number of halo rows
  auto halo_rows = [&](const Item& it, int& g0, int& rows) ICPP_INLINE {
    g0 = it.row0 / p.cW;
    rows = (min(it.row0 + BM, p.M) - 1) / p.cW - g0 + 3;
  };
  auto setup_halo = [&](const Item& it) ICPP_INLINE {
    if constexpr (HALO) {
      const int Wd = p.cW;
      int g0, rows;
      halo_rows(it, g0, rows);
      h_z = __builtin_amdgcn_readfirstlane(rows * Wd);
#pragma unroll
      for (int tm = 0; tm < G::TM; ++tm) {
        int m = it.row0 + wm * G::WTM + tm * MF + (lane % MF);
        m = min(m, p.M - 1);  // rows past M compute on a valid pixel and are never stored
        const int g = fdiv(m, p.dv_w);
        const int ow = m - g * Wd;
        const int oh = g - fdiv(g, p.dv_h) * p.cH;
        h_q[tm] = (g - g0) * Wd + ow - 1;
        const int rm = (oh > 0 ? 1 : 0) | 2 | (oh < p.cH - 1 ? 4 : 0);      // tap rows kh inside the image
        const int cm = (ow > 0 ? 1 : 0) | 2 | (ow < Wd - 1 ? 4 : 0);        // tap columns kw inside
        h_vmask[tm] = ((rm & 1) ? cm : 0) | ((rm & 2) ? cm << 3 : 0) | ((rm & 4) ? cm << 6 : 0);
      }
    }
  };
  auto issue_halo = [&](const Item& it) ICPP_INLINE {
    if constexpr (HALO) {
      const int Wd = p.cW;
      int g0, rows;
      halo_rows(it, g0, rows);
      const int zpix = rows * Wd;
      const int nslots = (zpix + 1) * 8;             // the launcher keeps nslots * 16 <= HALO_CAP
      // halo pixel q is input pixel (g0 - 1) * W + q of the N*H*W stacked pixels (rows
      // past the first or last image row of the batch load zeros)
      const int pix0 = (g0 - 1) * Wd;
#pragma unroll
      for (int i = 0; i < HL; ++i) {
        const int s = i * G::THREADS + tid;
        if (s < nslots) {
          const int q = s >> 3;
          const int pix = pix0 + q;
          const int chunk = (s & 7) ^ halo_swz(q);
          const bool ok = q < zpix && pix >= 0 && pix < p.M;
          const uint32_t off = ok ? (uint32_t)((pix * p.cC + chunk * 8) * ESZ) : p.a_bytes_total;
          dma16(ra, off, 0u, (char ICPP_LDS*)halo_lds + i * G::THREADS * 16 + wave_slot);
        }
      }
    }
  };
  const uint32_t a_row_step = (uint32_t)((G::THREADS / G::CPR_A) * p.lda * ESZ);  // bytes per load (A_UNIFORM)
  const uint32_t b_row_step = (uint32_t)((G::THREADS / G::CPR_B) * p.ldb * ESZ);  // bytes per load (B_UNIFORM)

  // Per-tile part of the A address shared by all loads of a K tile.  For the
  // per-tile-tap gather (C % BK == 0) that tile is filter tap `tap` and channels
  // c0 .. c0+BK-1 of it, and a lane's offset is its tap-(0,0) base plus the tile
  // constant toff, or past the buffer (zeros) when the tap falls in the padding.
  // The issue cursor carries (tap, filter column, c0, tap byte offset) from tile to
  // tile with adds and selects: one wave issues one instruction per 4 cycles, so
  // the two runtime divisions a K index -> (tap, c0) decomposition costs (~60
  // scalar instructions) would outlast the tile's MFMAs.
  struct TileCtx { int tap; int toff; };
  int t_tap = 0, t_kw = 0, t_c0 = 0, t_off = 0, t_col_step = 0, t_row_step = 0;
  if constexpr (TAPS) {
    const int kg = (first.kz * p.k_split) / BK;  // the item's first K tile
    const int tiles_per_tap = p.cC / BK;
    t_tap = kg / tiles_per_tap;
    t_c0 = (kg - t_tap * tiles_per_tap) * BK;
    const int kh = t_tap / p.cKW;
    t_kw = t_tap - kh * p.cKW;
    t_off = (kh * p.cD * p.cW + t_kw * p.cD) * p.cC * ESZ;
    t_col_step = p.cD * p.cC * ESZ;                              // (kh, kw) -> (kh, kw + 1)
    t_row_step = (p.cD * p.cW - (p.cKW - 1) * p.cD) * p.cC * ESZ;  // (kh, KW - 1) -> (kh + 1, 0)
    // wave-uniform by construction; said so, the scalar cursor below may hold them in SGPRs
    t_tap = __builtin_amdgcn_readfirstlane(t_tap);
    t_c0 = __builtin_amdgcn_readfirstlane(t_c0);
    t_kw = __builtin_amdgcn_readfirstlane(t_kw);
    t_off = __builtin_amdgcn_readfirstlane(t_off);
    t_col_step = __builtin_amdgcn_readfirstlane(t_col_step);
    t_row_step = __builtin_amdgcn_readfirstlane(t_row_step);
  }
  auto cursor_ctx = [&]() ICPP_INLINE { return TileCtx{t_tap, t_off + t_c0 * ESZ}; };
  // The tap cursor one K tile on.  Past the item's last tile it keeps going: the
  // issue index of B is clamped (a cached re-read), and A's tap runs past KH * KW
  // (at most STAGES - 1 taps, so below 32), whose mask bits are 0 -- those loads
  // take the out-of-range offset and return zeros, into stages nobody reads.
  // Written as scalar instructions: the state is wave-uniform, but compiled from C++
  // the compare-and-increment becomes a vector add-with-carry and the cursor moves
  // into VGPRs (~17 vector instructions per tile).  12 scalar ones here:
  //   c0 += BK; w = (c0 == C); c0 = w ? 0 : c0; tap += w; kw += w; off += w ? col : 0;
  //   r = (kw == KW); kw = r ? 0 : kw; off += r ? row - col : 0.
  const int t_rmc = t_row_step - t_col_step;
  auto cursor_step = [&]() ICPP_INLINE {
    if constexpr (TAPS) {
      int t1, w;
      asm volatile(
          "s_add_i32 %0, %0, %6\n\t"
          "s_cmp_eq_u32 %0, %7\n\t"
          "s_cselect_b32 %0, 0, %0\n\t"
          "s_cselect_b32 %4, %8, 0\n\t"
          "s_cselect_b32 %5, 1, 0\n\t"
          "s_add_i32 %1, %1, %5\n\t"
          "s_add_i32 %2, %2, %5\n\t"
          "s_add_i32 %3, %3, %4\n\t"
          "s_cmp_eq_u32 %2, %9\n\t"
          "s_cselect_b32 %2, 0, %2\n\t"
          "s_cselect_b32 %4, %10, 0\n\t"
          "s_add_i32 %3, %3, %4"
          : "+s"(t_c0), "+s"(t_tap), "+s"(t_kw), "+s"(t_off), "=&s"(t1), "=&s"(w)
          : "s"(BK), "s"(__builtin_amdgcn_readfirstlane(p.cC)), "s"(t_col_step),
            "s"(__builtin_amdgcn_readfirstlane(p.cKW)), "s"(__builtin_amdgcn_readfirstlane(t_rmc))
          : "scc");
    }
  };
  // One 16-byte-per-lane load of the tile at K element kk into stage S: loads
  // 0 .. SA-1 move A chunks, SA .. SA+SB-1 move B chunks.  Issued one at a time
  // so the mainloop can spread them between the MFMAs of the tile being multiplied.
  auto issue_load = [&](int kk, auto S, auto L, const TileCtx& tc, uint32_t boff) ICPP_INLINE {
    constexpr int l = decltype(L)::value;
    char ICPP_LDS* as = stage_base(S);
    char ICPP_LDS* bs = as + A_OFF;
    if constexpr (l < LA) {
      constexpr int i = l;
      if (!(G::A_EVEN || tid + i * G::THREADS < G::A_CHUNKS)) return;
      if constexpr (DENSE) {
        if constexpr (A_UNIFORM)
          dma16(ra, a_goff[0], (uint32_t)(kk * ESZ) + i * a_row_step, as + i * G::THREADS * 16 + wave_slot);
        else
          dma16(ra, a_goff[i], (uint32_t)(kk * ESZ), as + i * G::THREADS * 16 + wave_slot);
      } else if constexpr (TAPS) {
        const bool ok = (a_tmask[i] >> tc.tap) & 1u;  // tc.tap < 32
        const uint32_t off = ok ? (uint32_t)(a_tbase[i] + tc.toff) : p.a_bytes_total;
        dma16(ra, off, 0u, as + i * G::THREADS * 16 + wave_slot);
      } else {
        // K index of this chunk -> (kh, kw, c); one filter tap per chunk since C % 8 == 0
        const int k = kk + a_lc[i] * G::CH;
        const int tap = k / p.cC;
        const int ci = k - tap * p.cC;
        const int kh = tap / p.cKW, kw = tap - (tap / p.cKW) * p.cKW;
        const int ih = a_ih0[i] + kh * p.cD, iw = a_iw0[i] + kw * p.cD;
        const bool ok = a_img[i] >= 0 && ih >= 0 && ih < p.cH && iw >= 0 && iw < p.cW && k < p.K;
        const uint32_t off = ok ? (uint32_t)((((a_img[i] * p.cH + ih) * p.cW + iw) * p.cC + ci) * ESZ)
                                : (uint32_t)p.a_bytes_total;
        dma16(ra, off, 0u, as + i * G::THREADS * 16 + wave_slot);
      }
    } else {
      constexpr int i = l - LA;
      if (!(G::B_EVEN || tid + i * G::THREADS < G::B_CHUNKS)) return;
      if constexpr (B_UNIFORM)
        dma16(rb, b_goff[0], boff + i * b_row_step, bs + i * G::THREADS * 16 + wave_slot);
      else
        dma16(rb, b_goff[i], boff, bs + i * G::THREADS * 16 + wave_slot);
    }
  };
  constexpr int LOADS = LA + G::SB;  // loads per thread per tile
  // boff: byte offset of the tile's first B row (kk * ldb * ESZ)
  auto issue_tile = [&](int kk, auto S, const TileCtx& tc, uint32_t boff) ICPP_INLINE {
    static_for<LOADS>([&](auto L) ICPP_INLINE { issue_load(kk, S, L, tc, boff); });
  };

  Acc acc[G::TM][G::TN];
#pragma unroll
  for (int i = 0; i < G::TM; ++i)
#pragma unroll
    for (int j = 0; j < G::TN; ++j) acc[i][j] = Acc{};

  // ---- per-lane fragment addressing --------------------------------------
  // The swizzle term of a lane is the same for every MFMA tile row (tm) and
  // every K step row offset, so an address is (per-lane register) + (compile-
  // time immediate): A needs one register per K step, B one per N tile.
  constexpr int NKS = BK / G::KI;
  const int li = lane & 15;
  const int a_lrow = wm * G::WTM + (lane % MF);
  const int a_kgrp = lane / MF;                     // K slice of this lane: 0..3 (MF16) / 0..1 (MF32)
  // row bands of a wave are MF rows apart: with a swizzle period above MF, odd and even
  // bands take separate address sets
  constexpr int AP = (G::TM > 1 && G::A_SWZ_PERIOD > MF) ? 2 : 1;
  uint32_t a_addr[AP][NKS][ESZ == 2 ? 1 : 2];
#pragma unroll
  for (int par = 0; par < AP; ++par) {
    const int a_s = G::a_swz(a_lrow + par * MF);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      if constexpr (ESZ == 2) {
        const int c = (ks * G::KI) / 8 + a_kgrp;
        a_addr[par][ks][0] = (uint32_t)(a_lrow * G::ROWB_A + ((c ^ a_s) << 4));
      } else {
        const int c = (ks * G::KI) / 16 + a_kgrp * 2;
        a_addr[par][ks][0] = (uint32_t)(a_lrow * G::ROWB_A + ((c ^ a_s) << 4));
        a_addr[par][ks][1] = (uint32_t)(a_lrow * G::ROWB_A + (((c + 1) ^ a_s) << 4));
      }
    }
  }
  const int b_ncol_base = wn * G::WTN + ((MF == 32) ? 16 * ((lane >> 4) & 1) : 0);
  const int b_kgrp = (MF == 32) ? (lane >> 5) : (lane >> 4);
  uint32_t b_addr[G::TN];
#pragma unroll
  for (int tn = 0; tn < G::TN; ++tn) {
    const int n0 = b_ncol_base + tn * MF;
    if constexpr (ESZ == 2) {
      // tr16: lane i of a 16-lane group points at row k0 + i/4, columns n0 + 4*(i%4) .. +3
      const int k = b_kgrp * 8 + (li >> 2);
      const int col = n0 + 4 * (li & 3);
      b_addr[tn] = (uint32_t)(k * G::ROWB_B + (((col >> 3) ^ G::b_swz(k)) << 4) + (col & 7) * 2);
    } else {
      // tr8: lane i of a 16-lane group points at row k0 + i/2, columns n0 + 8*(i%2) .. +7
      const int k = b_kgrp * 32 + (li >> 1);
      const int col = n0 + 8 * (li & 1);
      b_addr[tn] = (uint32_t)(k * G::ROWB_B + (((col >> 4) ^ G::b_swz(k)) << 4) + (col & 15));
    }
  }

  auto load_frags = [&](const char ICPP_LDS* as, const char ICPP_LDS* bs, auto KS, Frag* af, Frag* bf,
                        int tap) ICPP_INLINE {
    constexpr int ks = decltype(KS)::value;
    // A_HALO: K tile `tap` of the tile is filter tap (kh, kw), which offsets the halo
    // pixel.  Per MFMA row band, pa = q * 128 + ((lane K chunk ^ swizzle(q)) << 4) is the
    // same for every K-step of the tile (computed once per tile); a K-step's first
    // chunk only XORs bits 4-6.
    const int t_tap = HALO ? tap : 0;
    const int t_kh = HALO ? t_tap / 3 : 0;
    const int t_off = HALO ? t_kh * p.cW + (t_tap - t_kh * 3) : 0;
    constexpr int h_chunk = (ks * G::KI) / 8;  // first 16-byte chunk of this K step
#pragma unroll
    for (int tm = 0; tm < G::TM; ++tm) {
      const uint32_t row_off = (uint32_t)(tm * MF * G::ROWB_A);
      if constexpr (HALO) {
        const int q = ((h_vmask[tm] >> t_tap) & 1) ? h_q[tm] + t_off : h_z;
        const uint32_t pa = ((uint32_t)q << 7) + (uint32_t)((a_kgrp ^ halo_swz(q)) << 4);
        // this K-step's first chunk has the lane chunk bits clear: an XOR of bits 4-6
        af[tm] = lds_load16((const char ICPP_LDS*)halo_lds, pa ^ (uint32_t)(h_chunk << 4));
      } else if constexpr (ESZ == 2) {
        af[tm] = lds_load16(as, a_addr[tm % AP][ks][0] + row_off);
      } else {
        i32x4 lo = lds_load16(as, a_addr[tm % AP][ks][0] + row_off);
        i32x4 hi = lds_load16(as, a_addr[tm % AP][ks][1] + row_off);
        af[tm] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
    }
#pragma unroll
    for (int tn = 0; tn < G::TN; ++tn) {
      if constexpr (ESZ == 2) {
        const uint32_t k_off = (uint32_t)(ks * G::KI * G::ROWB_B);
        i32x2 lo = lds_tr16(bs, b_addr[tn] + k_off);
        i32x2 hi = lds_tr16(bs, b_addr[tn] + k_off + 4 * G::ROWB_B);
        bf[tn] = i32x4{lo[0], lo[1], hi[0], hi[1]};
      } else {
        i32x2 v[4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          v[rr] = lds_tr8(bs, b_addr[tn] + (uint32_t)((ks * G::KI + 8 * rr) * G::ROWB_B));
        bf[tn] = i32x8{v[0][0], v[0][1], v[1][0], v[1][1], v[2][0], v[2][1], v[3][0], v[3][1]};
      }
    }
  };

  // ---- pipelined mainloop --------------------------------------------------
  // The K dimension is a stream of MFMA K-steps (NKS per tile).  The fragments
  // of step s+1 are read from LDS while the MFMAs of step s issue, across tile
  // boundaries too, so a wave never waits on LDS latency at the start of a
  // tile.  The LDS ring holds STAGES tiles.  Barrier B(kt) sits before the last
  // K-step of tile kt: by then every wave has read all fragments of tile kt
  // (they were read during the previous step), so B(kt) both publishes tile
  // kt+1 (each wave first waits for its own loads of it) and retires stage
  // kt % STAGES, which is refilled at once with tile kt+STAGES.  After the
  // barrier the wave goes straight to MFMAs on fragments already in registers.
  //
  // Past the last tile the fetch index is clamped to nk-1 (a re-read of a
  // cached tile into a stage nobody reads again), so every step issues exactly
  // LOADS loads and the vmcnt threshold is a constant.
  constexpr int DS_PER_KS = G::TM * (ESZ == 2 ? 1 : 2) + G::TN * (ESZ == 2 ? 2 : 4);
  constexpr int MFMA_PER_KS = G::TM * G::TN;
  static_assert(PP || (STAGES * NKS) % 2 == 0, "fragment double buffer parity must repeat every STAGES tiles");
  // Loads this wave issues per tile.  Tile loads cover whole waves (chunk
  // counts are multiples of 64), so in the last, partial round of A or B loads
  // a wave either loads or skips as a whole: per wave the count is LOADS,
  // LOADS-1 or LOADS-2, and vmcnt thresholds follow it.
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const int my_loads = (!HALO && G::A_CHUNKS > 64 * wv ? (G::A_CHUNKS - 64 * wv + G::THREADS - 1) / G::THREADS : 0) +
                       (G::B_CHUNKS > 64 * wv ? (G::B_CHUNKS - 64 * wv + G::THREADS - 1) / G::THREADS : 0);
  // s_waitcnt vmcnt(TILES * my_loads): at most TILES tiles of this wave's loads still in flight
  auto wait_tiles = [&](auto TILES) ICPP_INLINE {
    constexpr int nt = decltype(TILES)::value;
    if constexpr (nt == 0 || ((HALO || G::A_EVEN) && G::B_EVEN)) {
      wait_vmcnt<nt * LOADS>();
    } else {
      if (my_loads == LOADS) wait_vmcnt<nt * LOADS>();
      else if (my_loads == LOADS - 1) wait_vmcnt<nt * (LOADS - 1)>();
      else wait_vmcnt<nt * (LOADS >= 2 ? LOADS - 2 : 0)>();
    }
  };

  Frag fa[2][G::TM], fb[2][G::TN];
  auto mfma_step = [&](const Frag* af, const Frag* bf) ICPP_INLINE {
#pragma unroll
    for (int tm = 0; tm < G::TM; ++tm)
#pragma unroll
      for (int tn = 0; tn < G::TN; ++tn) acc[tm][tn] = Op::run(bf[tn], af[tm], acc[tm][tn]);
  };
  // Issue order for the scheduler within one K-step: its MFMAs one by one, with
  // the next step's fragment reads (left alone, the backend re-reads fragments
  // just before use and waits on each) and NL tile loads (issued as one burst
  // they stall the wave on the vector-memory queue -- the CU's texture path
  // takes ~16 cycles per 1 KiB load -- ahead of its MFMAs) spread between the
  // first SPAN of them, so the reads have landed by the next barrier.
  auto schedule = [&](auto NL) ICPP_INLINE {
    constexpr int nl_total = decltype(NL)::value;
    constexpr int SPAN = (MFMA_PER_KS * 3) / 4 > 0 ? (MFMA_PER_KS * 3) / 4 : 1;
    static_for<MFMA_PER_KS>([&](auto I) ICPP_INLINE {
      constexpr int i = decltype(I)::value;
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      // items x with floor(x * SPAN / total) == i follow MFMA i
      constexpr int ds = (i < SPAN) ? ((i + 1) * DS_PER_KS + SPAN - 1) / SPAN - (i * DS_PER_KS + SPAN - 1) / SPAN : 0;
      if constexpr (ds > 0) __builtin_amdgcn_sched_group_barrier(0x100, ds, 0);
      constexpr int nl = (i < SPAN) ? ((i + 1) * nl_total + SPAN - 1) / SPAN - (i * nl_total + SPAN - 1) / SPAN : 0;
      if constexpr (nl > 0) __builtin_amdgcn_sched_group_barrier(0x020, nl, 0);
    });
  };

  // ---- epilogue of one item ----
  auto epilogue = [&](const Item& it) ICPP_INLINE {
    const int row0 = it.row0, col0 = it.col0, kz = it.kz;
    // lane owns output row (lane % MF) of each MFMA tile and groups of 4 consecutive columns
    constexpr int NG = Op::ACC / 4;  // column groups per MFMA tile
    auto out_row = [&](int tm) ICPP_INLINE { return row0 + wm * G::WTM + tm * MF + (lane % MF); };
    auto out_col = [&](int tn, int g) ICPP_INLINE {
      return col0 + wn * G::WTN + tn * MF + ((MF == 16) ? 4 * (lane >> 4) : (8 * g + 4 * (lane >> 5)));
    };
    auto get4 = [&](int tm, int tn, int g) ICPP_INLINE {
      return f32x4{acc[tm][tn][4 * g + 0], acc[tm][tn][4 * g + 1], acc[tm][tn][4 * g + 2], acc[tm][tn][4 * g + 3]};
    };

    // Output through LDS: for each MFMA row band (tm) a wave writes its values
    // (converted to OutT) into a private padded LDS region, then re-reads them as
    // 16-byte row chunks, so global stores cover whole contiguous row segments
    // instead of 8-byte pieces of 16 different rows.
    // With a residual (RES), each band's residual rows are read the same way --
    // 16-byte row chunks, the next band's loads in flight while the current one
    // is computed -- written into the band's LDS region, and read back by each
    // lane in the accumulator layout before it overwrites them with its outputs.
    auto store_staged_impl = [&](auto RES, const OutT* res, auto&& value4) ICPP_INLINE {
      constexpr bool HAS_RES = decltype(RES)::value;
      constexpr int OSZ = (int)sizeof(OutT);
      constexpr int ROWB_O = G::WTN * OSZ + 16;           // +16 B rotates rows across banks
      constexpr int REGION = MF * ROWB_O;
      constexpr int CPR_O = G::WTN * OSZ / 16;             // 16-byte chunks per output row
      constexpr int CHUNK_ELEMS = 16 / OSZ;
      constexpr int NQ = (MF * CPR_O + 63) / 64;           // chunks per lane per band
      // staging space: the pipeline stage arrays, or for A_HALO the halo (free after the mainloop)
      constexpr int PER_STAGE = (HALO ? HALO_CAP : SBYTES) / REGION;  // wave regions per array
      static_assert(PER_STAGE * (HALO ? 1 : STAGES) >= WM * WN, "epilogue staging must fit the LDS stages");
      static_assert((G::WTN * OSZ) % 16 == 0, "wave tile rows must be whole 16-byte chunks");
      // store descriptor over this tile's rows (launchers keep BM * ldc * OSZ < 2 GiB)
      const uint64_t rows = (uint64_t)(p.M > row0 ? min(p.M - row0, BM) : 0);
      const __amdgpu_buffer_rsrc_t rc = make_rsrc((OutT*)p.C + (size_t)row0 * p.ldc, (uint32_t)(rows * p.ldc * OSZ));
      // chunk j of a band: its (row, 16-byte column) in the wave tile and byte offset in the tile's rows
      auto chunk_off = [&](int tm, int q) ICPP_INLINE {
        const int rr = q / CPR_O, cc = q % CPR_O;
        const int r = wm * G::WTM + tm * MF + rr;  // row within the tile: rows >= M lie past the range
        const int n = col0 + wn * G::WTN + cc * CHUNK_ELEMS;
        return n < p.N ? (uint32_t)(r * p.ldc + n) * OSZ : ICPP_OOB_OFFSET;
      };
      // With few bands every band's residual goes out at once, before the barrier
      // (one memory latency instead of one per band); otherwise the next band's
      // loads are in flight while the current band is computed.
      constexpr bool RES_ALL = HAS_RES && G::TM * NQ <= 8;
      i32x4 rnext[NQ];
      i32x4 rall[RES_ALL ? G::TM : 1][NQ];
      __amdgpu_buffer_rsrc_t rr_src;
      auto load_band_to = [&](int tm, i32x4 (&dst)[NQ]) ICPP_INLINE {
#pragma unroll
        for (int j = 0; j < NQ; ++j) {
          const int q = j * 64 + lane;
          // past the range (rows >= M, columns >= N): the hardware returns zeros
          dst[j] = ((MF * CPR_O) % 64 == 0 || q < MF * CPR_O)
                       ? __builtin_amdgcn_raw_buffer_load_b128(rr_src, chunk_off(tm, q), 0, 0)
                       : i32x4{0, 0, 0, 0};
        }
      };
      auto load_band = [&](int tm) ICPP_INLINE { load_band_to(tm, rnext); };
      if constexpr (HAS_RES) {
        rr_src = make_rsrc(res + (size_t)row0 * p.ldc, (uint32_t)(rows * p.ldc * OSZ));
        if constexpr (RES_ALL) {
#pragma unroll
          for (int tm = 0; tm < G::TM; ++tm) load_band_to(tm, rall[tm]);
        } else {
          load_band(0);
        }
      }
      const int w_arr = wave / PER_STAGE;
      char ICPP_LDS* arr = HALO ? (char ICPP_LDS*)halo_lds
                         : (w_arr == 0) ? (char ICPP_LDS*)lds0 : (w_arr == 1) ? (char ICPP_LDS*)lds1
                         : (w_arr == 2) ? (char ICPP_LDS*)lds2 : (char ICPP_LDS*)lds3;
      char ICPP_LDS* region = arr + (wave % PER_STAGE) * REGION;
      __syncthreads();  // every wave is done reading the pipeline stages
#pragma unroll
      for (int tm = 0; tm < G::TM; ++tm) {
        if constexpr (HAS_RES) {
          i32x4 rcur[NQ];
          if constexpr (RES_ALL) {
#pragma unroll
            for (int j = 0; j < NQ; ++j) rcur[j] = rall[tm][j];
          } else {
#pragma unroll
            for (int j = 0; j < NQ; ++j) rcur[j] = rnext[j];
            if (tm + 1 < G::TM) load_band(tm + 1);
          }
#pragma unroll
          for (int j = 0; j < NQ; ++j) {
            const int q = j * 64 + lane;
            if ((MF * CPR_O) % 64 == 0 || q < MF * CPR_O)
              *(i32x4 ICPP_LDS*)(region + (q / CPR_O) * ROWB_O + (q % CPR_O) * 16) = rcur[j];
          }
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
          __builtin_amdgcn_wave_barrier();
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
#pragma unroll
        for (int tn = 0; tn < G::TN; ++tn)
#pragma unroll
          for (int g = 0; g < NG; ++g) {
            const int lcol = tn * MF + ((MF == 16) ? 4 * (lane >> 4) : (8 * g + 4 * (lane >> 5)));
            char ICPP_LDS* at = region + (lane % MF) * ROWB_O + lcol * OSZ;
            f32x4 r = {0.f, 0.f, 0.f, 0.f};
            if constexpr (HAS_RES) r = Vec4Store<OutT>::ld_lds(at);  // this lane's own elements
            Vec4Store<OutT>::st_lds(at, value4(tm, tn, g, r));
          }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int j = 0; j < NQ; ++j) {
          const int q = j * 64 + lane;
          if ((MF * CPR_O) % 64 == 0 || q < MF * CPR_O) {
            const i32x4 v = *(const i32x4 ICPP_LDS*)(region + (q / CPR_O) * ROWB_O + (q % CPR_O) * 16);
            buf_store16(rc, chunk_off(tm, q), v);
          }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
    };
    auto store_staged = [&](auto&& value4) ICPP_INLINE {
      store_staged_impl(std::false_type{}, nullptr,
                        [&](int tm, int tn, int g, f32x4) ICPP_INLINE { return value4(tm, tn, g); });
    };

    // a row's sum over this wave's columns, reduced across the lanes sharing the row
    auto lane_reduce = [&](float v) ICPP_INLINE {
      if (MF == 16) {
        v += __shfl_xor(v, 16);
        v += __shfl_xor(v, 32);
      } else {
        v += __shfl_xor(v, 32);
      }
      return v;
    };
    if constexpr (EPI == EPI_STORE) {
      if (p.partial) {
        float* ws = p.ws + (size_t)kz * p.M * p.N;
#pragma unroll
        for (int tm = 0; tm < G::TM; ++tm) {
          const int m = out_row(tm);
#pragma unroll
          for (int tn = 0; tn < G::TN; ++tn)
#pragma unroll
            for (int g = 0; g < NG; ++g) {
              const int n = out_col(tn, g);
              if (m < p.M && n < p.N) Vec4Store<float>::st(ws + (size_t)m * p.N + n, get4(tm, tn, g));
            }
        }
      } else if (!DENSE && p.ce.flags != 0) {
        // fused conv epilogue (reference conv2d_bn / conv2d_bn_relu / conv_bn_add_relu)
        if constexpr (!DENSE) {
          f32x4 sc[G::TN][NG], sh[G::TN][NG];
#pragma unroll
          for (int tn = 0; tn < G::TN; ++tn)
#pragma unroll
            for (int g = 0; g < NG; ++g) conv_bn4<BiasT>(p.ce, p.N, out_col(tn, g), sc[tn][g], sh[tn][g]);
          auto run = [&](auto RES) ICPP_INLINE {
            dispatch_relu(p.act, [&](auto ACT) ICPP_INLINE {
              store_staged_impl(RES, (const OutT*)p.ce.residual, [&](int tm, int tn, int g, f32x4 r) ICPP_INLINE {
                return conv_epi4<decltype(ACT)::value, OutT>(get4(tm, tn, g), sc[tn][g], sh[tn][g], r);
              });
            });
          };
          if (p.ce.flags & CEPI_RESIDUAL) run(std::true_type{});
          else run(std::false_type{});
        }
      } else {
        const __amdgpu_buffer_rsrc_t bias_r = vec_rsrc<BiasT>(p.bias, p.N);
        f32x4 bv[G::TN][NG];
#pragma unroll
        for (int tn = 0; tn < G::TN; ++tn)
#pragma unroll
          for (int g = 0; g < NG; ++g) bv[tn][g] = Vec4Ld<BiasT>::ld(bias_r, out_col(tn, g));
        // LayerNorm producer (p.stat_cols > 0, act none): each row's values over this
        // wave's WTN columns are stored minus their mean, and the mean goes to
        // ws[m * stat_cols + column block] in fp32.  The LayerNorm pass adds it back,
        // so the 16-bit copy carries only the spread around the block mean: a row whose
        // mean is far from zero keeps the fp32 precision the reference's X has.
        float bmean[G::TM];
#pragma unroll
        for (int tm = 0; tm < G::TM; ++tm) bmean[tm] = 0.f;
        if (p.stat_cols > 0) {
          const int wcol0 = col0 + wn * G::WTN;
          const int wcnt = max(0, min(G::WTN, p.N - wcol0));
          const int scol = wcol0 / G::WTN;
#pragma unroll
          for (int tm = 0; tm < G::TM; ++tm) {
            float s = 0.f;
#pragma unroll
            for (int tn = 0; tn < G::TN; ++tn)
#pragma unroll
              for (int g = 0; g < NG; ++g) {
                const f32x4 v = get4(tm, tn, g);
                if (out_col(tn, g) < p.N)
#pragma unroll
                  for (int e = 0; e < 4; ++e) s += v[e] * p.alpha + bv[tn][g][e];
              }
            s = lane_reduce(s);
            bmean[tm] = wcnt > 0 ? s / (float)wcnt : 0.f;
            const int m = out_row(tm);
            if (lane < MF && m < p.M && scol < p.stat_cols) p.ws[(size_t)m * p.stat_cols + scol] = bmean[tm];
          }
        }
        dispatch_act(p.act, [&](auto ACT) ICPP_INLINE {
          store_staged([&](int tm, int tn, int g) ICPP_INLINE {
            f32x4 v = get4(tm, tn, g);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = act_fn<decltype(ACT)::value>(v[e] * p.alpha + bv[tn][g][e]) - bmean[tm];
            return v;
          });
        });
      }
    } else {
      // LayerNorm epilogues: x = acc + bias (+ residual), statistics over valid columns (n < N)
      OutT* C = (OutT*)p.C;
      const __amdgpu_buffer_rsrc_t bias_r = vec_rsrc<BiasT>(p.bias, p.N);
      const OutT* res = (const OutT*)p.residual;
      float xs[G::TM][G::TN][Op::ACC];
#pragma unroll
      for (int tn = 0; tn < G::TN; ++tn)
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          const int n = out_col(tn, g);
          const f32x4 bv = Vec4Ld<BiasT>::ld(bias_r, n);
          const bool ok = n < p.N;
#pragma unroll
          for (int tm = 0; tm < G::TM; ++tm)
#pragma unroll
            for (int e = 0; e < 4; ++e) xs[tm][tn][4 * g + e] = ok ? (acc[tm][tn][4 * g + e] + bv[e]) : 0.f;
        }
      if (res != nullptr) {
        // one row band's loads at a time (a scheduling barrier per band): the largest
        // tiles have no registers left for every band's residual in flight.  Rows past M
        // and columns past N read zeros from the descriptor over the tile's rows.
        const uint32_t res_rows = (uint32_t)(p.M > row0 ? min(p.M - row0, BM) : 0);
        const __amdgpu_buffer_rsrc_t res_r =
            make_rsrc(res + (size_t)row0 * p.ldc, res_rows * (uint32_t)p.ldc * (uint32_t)sizeof(OutT));
#pragma unroll
        for (int tm = 0; tm < G::TM; ++tm) {
          const int r = out_row(tm) - row0;
#pragma unroll
          for (int tn = 0; tn < G::TN; ++tn)
#pragma unroll
            for (int g = 0; g < NG; ++g) {
              const int n = out_col(tn, g);
              const uint32_t off = n < p.N ? (uint32_t)(r * p.ldc + n) * (uint32_t)sizeof(OutT) : ICPP_OOB_OFFSET;
              const f32x4 rv = Vec4Ld<OutT>::at(res_r, off);
#pragma unroll
              for (int e = 0; e < 4; ++e) xs[tm][tn][4 * g + e] += rv[e];
            }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      const int wcol0 = col0 + wn * G::WTN;
      const int wcnt = max(0, min(G::WTN, p.N - wcol0));
      if constexpr (EPI == EPI_LN_STATS) {
        float* ws = p.ws;
        const int scol = wcol0 / G::WTN;
#pragma unroll
        for (int tm = 0; tm < G::TM; ++tm) {
          float s = 0.f;
#pragma unroll
          for (int tn = 0; tn < G::TN; ++tn)
#pragma unroll
            for (int e = 0; e < Op::ACC; ++e) s += xs[tm][tn][e];
          s = lane_reduce(s);
          const float mean = wcnt > 0 ? s / (float)wcnt : 0.f;
          float q = 0.f;
#pragma unroll
          for (int tn = 0; tn < G::TN; ++tn)
#pragma unroll
            for (int g = 0; g < NG; ++g) {
              const bool ok = out_col(tn, g) < p.N;
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const float d = xs[tm][tn][4 * g + e] - mean;
                q += ok ? d * d : 0.f;
              }
            }
          q = lane_reduce(q);
          const int m = out_row(tm);
          if (lane < MF && m < p.M && scol < p.stat_cols) {
            ws[((size_t)m * p.stat_cols + scol) * 2 + 0] = mean;
            ws[((size_t)m * p.stat_cols + scol) * 2 + 1] = q;
          }
          // X is stored centred on the block mean (the finalize adds it back), so the
          // 16-bit copy keeps the precision of the fp32 values whatever the row's offset
#pragma unroll
          for (int tn = 0; tn < G::TN; ++tn)
#pragma unroll
            for (int g = 0; g < NG; ++g) {
              const int n = out_col(tn, g);
              f32x4 v = {xs[tm][tn][4 * g] - mean, xs[tm][tn][4 * g + 1] - mean, xs[tm][tn][4 * g + 2] - mean,
                         xs[tm][tn][4 * g + 3] - mean};
              if (m < p.M && n < p.N) Vec4Store<OutT>::st(C + (size_t)m * p.ldc + n, v);
            }
        }
      } else if constexpr (EPI == EPI_LN_ROW) {
        // EPI_LN_ROW: the workgroup owns whole rows (tiles_n == 1, N <= BN); two-pass
        // mean / centred variance in registers, cross-wave through LDS.
        __syncthreads();  // mainloop LDS no longer needed
        static_assert(2 * WN * BM * 4 <= SBYTES, "LN reduction scratch must fit one LDS stage");
        float ICPP_LDS* red = (float ICPP_LDS*)lds0;       // [WN][BM]
        float ICPP_LDS* red2 = red + WN * BM;               // [WN][BM]
        const __amdgpu_buffer_rsrc_t gamma_r = vec_rsrc<BiasT>(p.gamma, p.N);
        const __amdgpu_buffer_rsrc_t beta_r = vec_rsrc<BiasT>(p.beta, p.N);
        const float inv_n = 1.f / (float)p.N;
        float mean[G::TM], rstd[G::TM];
#pragma unroll
        for (int tm = 0; tm < G::TM; ++tm) {
          float s = 0.f;
#pragma unroll
          for (int tn = 0; tn < G::TN; ++tn)
#pragma unroll
            for (int e = 0; e < Op::ACC; ++e) s += xs[tm][tn][e];
          s = lane_reduce(s);
          if (lane < MF) red[wn * BM + wm * G::WTM + tm * MF + lane] = s;
        }
        __syncthreads();
#pragma unroll
        for (int tm = 0; tm < G::TM; ++tm) {
          float s = 0.f;
          const int lr = wm * G::WTM + tm * MF + (lane % MF);
#pragma unroll
          for (int w = 0; w < WN; ++w) s += red[w * BM + lr];
          mean[tm] = s * inv_n;
          float q = 0.f;
#pragma unroll
          for (int tn = 0; tn < G::TN; ++tn)
#pragma unroll
            for (int g = 0; g < NG; ++g) {
              const bool ok = out_col(tn, g) < p.N;
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const float d = xs[tm][tn][4 * g + e] - mean[tm];
                q += ok ? d * d : 0.f;
              }
            }
          q = lane_reduce(q);
          if (lane < MF) red2[wn * BM + lr] = q;
        }
        __syncthreads();
#pragma unroll
        for (int tm = 0; tm < G::TM; ++tm) {
          float q = 0.f;
          const int lr = wm * G::WTM + tm * MF + (lane % MF);
#pragma unroll
          for (int w = 0; w < WN; ++w) q += red2[w * BM + lr];
          rstd[tm] = rsqrtf(q * inv_n + p.eps);
        }
#pragma unroll
        for (int tn = 0; tn < G::TN; ++tn)
#pragma unroll
          for (int g = 0; g < NG; ++g) {
            const int n = out_col(tn, g);
            const f32x4 gv = Vec4Ld<BiasT>::ld(gamma_r, n);
            const f32x4 bv = Vec4Ld<BiasT>::ld(beta_r, n);
            if (n >= p.N) continue;
#pragma unroll
            for (int tm = 0; tm < G::TM; ++tm) {
              const int m = out_row(tm);
              f32x4 v;
#pragma unroll
              for (int e = 0; e < 4; ++e) v[e] = (xs[tm][tn][4 * g + e] - mean[tm]) * rstd[tm] * gv[e] + bv[e];
              if (m < p.M) Vec4Store<OutT>::st(C + (size_t)m * p.ldc + n, v);
            }
          }
      } else {
        // EPI_LN_CR (co-resident row blocks): the launcher sizes every launch so that all
        // of its workgroups are resident at once.  The tiles_n workgroups of a row block
        // each publish their rows' (mean, M2) over their own columns to ws[m][tile column],
        // count themselves in on the row block's arrival counter and wait until all
        // tiles_n have; each then merges the row's tiles_n pairs in column order (Chan et
        // al., so the result does not depend on arrival order) and normalises its tile
        // from registers.  X never goes to memory and there is no second pass.
        // ln_ctr[2 rb] counts arrivals and ln_ctr[2 rb + 1] departures; the last
        // workgroup to depart zeroes both, so a call leaves the counters zero as it found
        // them.  A wait that runs out (workgroups not co-resident) sets *ln_err.
        // Everything that crosses workgroups -- the pairs and the counters -- goes through
        // device-scope stores and loads (sc1) and device atomics, which bypass the
        // per-XCD L2s' non-coherent copies, so no L2 write-back or invalidate is needed
        // (an agent-scope release fence here, an L2 write-back per wave, cost more than
        // the whole second pass it removes): each wave's pair stores complete (vmcnt 0)
        // before the barrier ahead of the arrival count, and the pair loads issue after
        // the barrier behind the observed count.
        static_assert(STAGES >= 2, "EPI_LN_CR keeps per-row results in the second stage array");
        constexpr int LN_CR_SPINS = 1 << 17;  // ~0.1-0.3 s of polling before giving up
        __syncthreads();  // every wave is done with the mainloop's LDS
        float ICPP_LDS* red = (float ICPP_LDS*)lds0;  // [WN][BM] per-wave row sums, then M2
        const int tcnt = max(0, min(BN, p.N - col0));
        const float inv_t = tcnt > 0 ? 1.f / (float)tcnt : 0.f;
        float tmean[G::TM];
#pragma unroll
        for (int tm = 0; tm < G::TM; ++tm) {
          float sum = 0.f;
#pragma unroll
          for (int tn = 0; tn < G::TN; ++tn)
#pragma unroll
            for (int e = 0; e < Op::ACC; ++e) sum += xs[tm][tn][e];  // zero past N
          sum = lane_reduce(sum);
          if (lane < MF) red[wn * BM + wm * G::WTM + tm * MF + lane] = sum;
        }
        __syncthreads();
#pragma unroll
        for (int tm = 0; tm < G::TM; ++tm) {
          const int lr = wm * G::WTM + tm * MF + (lane % MF);
          float sum = 0.f;
#pragma unroll
          for (int w = 0; w < WN; ++w) sum += red[w * BM + lr];
          tmean[tm] = sum * inv_t;
        }
        __syncthreads();  // red is reused for M2
#pragma unroll
        for (int tm = 0; tm < G::TM; ++tm) {
          float q = 0.f;
#pragma unroll
          for (int tn = 0; tn < G::TN; ++tn)
#pragma unroll
            for (int g = 0; g < NG; ++g) {
              const bool ok = out_col(tn, g) < p.N;
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const float d = xs[tm][tn][4 * g + e] - tmean[tm];
                q += ok ? d * d : 0.f;
              }
            }
          q = lane_reduce(q);
          if (lane < MF) red[wn * BM + wm * G::WTM + tm * MF + lane] = q;
        }
        __syncthreads();
        const int rb = row0 / BM, tcol = col0 / BN;
        if (wn == 0) {
#pragma unroll
          for (int tm = 0; tm < G::TM; ++tm) {
            const int lr = wm * G::WTM + tm * MF + (lane % MF);
            float q = 0.f;
#pragma unroll
            for (int w = 0; w < WN; ++w) q += red[w * BM + lr];
            const int m = out_row(tm);
            if (lane < MF && m < p.M) {
              float* dst = p.ws + ((size_t)m * p.tiles_n + tcol) * 2;
              __hip_atomic_store(dst, tmean[tm], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              __hip_atomic_store(dst + 1, q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
          }
          __builtin_amdgcn_s_waitcnt(0);  // this wave's pair stores have completed
        }
        __syncthreads();
        if (tid == 0) {
          int* ctr = p.ln_ctr + 2 * rb;
          __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          int spins = 0;
          while (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < p.tiles_n) {
            if (++spins > LN_CR_SPINS) {
              __hip_atomic_store(p.ln_err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              break;
            }
            __builtin_amdgcn_s_sleep(2);
          }
          // this workgroup no longer reads the arrival counter; the last to leave resets the pair
          if (__hip_atomic_fetch_add(ctr + 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == p.tiles_n - 1) {
            __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(ctr + 1, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        }
        __syncthreads();
        // The row block's pairs are one contiguous [rows][tiles_n][2] block of ws: 16-byte
        // device-scope loads spread over the workgroup bring it into LDS -- rows [0, r0) into
        // the first stage array, the rest into the second (r0 even, so the split falls on a
        // 16-byte boundary; the launcher checks that both parts fit) -- then one thread per
        // row merges its row and leaves the merged (mean, rstd) in the row's first pair.
        const int rows = max(0, min(BM, p.M - row0));
        const int prow = 2 * p.tiles_n;                                   // floats per row
        const int r0 = min(rows, (SBYTES / (4 * prow)) & ~1);
        auto row_pairs = [&](int r) ICPP_INLINE {
          return r < r0 ? (float ICPP_LDS*)lds0 + r * prow : (float ICPP_LDS*)lds1 + (r - r0) * prow;
        };
        {
          const int nvec = rows * p.tiles_n / 2;  // 16-byte vectors: two pairs each
          const int nvec0 = r0 * p.tiles_n / 2;   // those of rows [0, r0), exactly (r0 even)
          const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.ws + (size_t)row0 * p.tiles_n * 2, (uint32_t)(nvec * 16));
          for (int i = tid; i < nvec; i += G::THREADS) {
            char ICPP_LDS* dst = i < nvec0 ? (char ICPP_LDS*)lds0 + 16 * i : (char ICPP_LDS*)lds1 + 16 * (i - nvec0);
            *(i32x4 ICPP_LDS*)dst = __builtin_amdgcn_raw_buffer_load_b128(rs, (uint32_t)(i * 16), 0, 16);
          }
          if ((rows * p.tiles_n) & 1) {  // an odd last pair (odd tiles_n and an odd row count)
            if (tid == 0) {
              const int j = rows * p.tiles_n - 1;
              float ICPP_LDS* dst = row_pairs(rows - 1) + 2 * (p.tiles_n - 1);
              dst[0] = __hip_atomic_load(p.ws + ((size_t)row0 * p.tiles_n + j) * 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              dst[1] = __hip_atomic_load(p.ws + ((size_t)row0 * p.tiles_n + j) * 2 + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
          }
          __syncthreads();
          for (int r = tid; r < rows; r += G::THREADS) {
            float ICPP_LDS* pr = row_pairs(r);
            float n_acc = 0.f, mu = 0.f, m2 = 0.f;
            for (int j = 0; j < p.tiles_n; ++j) {
              const float nb = (float)max(0, min(BN, p.N - j * BN));
              const float mb = pr[2 * j + 0];
              const float qb = pr[2 * j + 1];
              const float nt = n_acc + nb;
              const float d = mb - mu;
              mu += d * (nb / nt);
              m2 += qb + d * d * (n_acc * nb / nt);
              n_acc = nt;
            }
            pr[0] = mu;  // this thread alone reads and writes row r
            pr[1] = rsqrtf(m2 / (float)p.N + p.eps);
          }
          __syncthreads();
        }
        const __amdgpu_buffer_rsrc_t gamma_r = vec_rsrc<BiasT>(p.gamma, p.N);
        const __amdgpu_buffer_rsrc_t beta_r = vec_rsrc<BiasT>(p.beta, p.N);
        f32x4 gv[G::TN][NG], bt[G::TN][NG];
#pragma unroll
        for (int tn = 0; tn < G::TN; ++tn)
#pragma unroll
          for (int g = 0; g < NG; ++g) {
            gv[tn][g] = Vec4Ld<BiasT>::ld(gamma_r, out_col(tn, g));
            bt[tn][g] = Vec4Ld<BiasT>::ld(beta_r, out_col(tn, g));
          }
        float mean[G::TM], rstd[G::TM];
#pragma unroll
        for (int tm = 0; tm < G::TM; ++tm) {
          const int lr = wm * G::WTM + tm * MF + (lane % MF);
          // rows past M (never stored) take the last valid row's values: every read stays
          // inside the pairs' region
          const float ICPP_LDS* pr = row_pairs(min(lr, rows - 1));
          mean[tm] = pr[0];
          rstd[tm] = pr[1];
        }
        store_staged([&](int tm, int tn, int g) ICPP_INLINE {
          f32x4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = (xs[tm][tn][4 * g + e] - mean[tm]) * rstd[tm] * gv[tn][g][e] + bt[tn][g][e];
          return v;
        });
      }
    }
  };

  // Issue cursor: the K tile issued last.  Past the last tile it stays there (a
  // cached re-read into a stage nobody reads again), so every step issues
  // exactly LOADS loads.
  int cur_kt = 0;
  // Conv tiles: the B byte offset of the issue cursor, advanced by one tile of rows
  // without the clamp (past K the loads fall outside B's range and return zeros;
  // past a split-K slice they read the next slice's rows; either lands in a stage
  // nobody reads).  Dense tiles compute it from the clamped cursor.
  uint32_t t_boff = (uint32_t)(first.kz * p.k_split * p.ldb * ESZ);
  const uint32_t t_bstep = (uint32_t)(BK * p.ldb * ESZ);
  auto advance_issue = [&]() ICPP_INLINE {
    cur_kt = min(cur_kt + 1, nk - 1);
    cursor_step();
    if constexpr (!DENSE) t_boff += t_bstep;
  };
  auto cur_kk = [&]() ICPP_INLINE { return first.kz * p.k_split + cur_kt * BK; };
  auto cur_boff = [&]() ICPP_INLINE {
    if constexpr (DENSE) return (uint32_t)(cur_kk() * p.ldb * ESZ);
    else return t_boff;
  };

  // K tile -> filter tap for A_HALO (C == BK: the K tiles are the taps; clamped for the
  // prefetch past the last tile, whose fragments are never used)
  const int kt_base = (first.kz * p.k_split) / BK;
  auto tap_of = [&](int kt) ICPP_INLINE { return HALO ? min(kt_base + kt, 8) : 0; };
  setup_halo(first);
  issue_halo(first);  // older than every B load: landed once tile 0 has
  if constexpr (PP) {
    // ---- ping-pong mainloop ----------------------------------------------------
    // Waves w and w + 4 share a SIMD, and group g = wm holds one wave per SIMD.
    // Every phase ends with one workgroup barrier.  In phase 2j group 0 reads the
    // fragments of tile j (memory phase) while group 1 multiplies tile j-1 (MFMA
    // phase); in phase 2j+1 group 0 multiplies tile j while group 1 reads it.  On
    // each SIMD one wave streams MFMAs from registers while the other fetches, so
    // the two no longer split the matrix core and then wait for each other at the
    // tile barrier.
    // Tile loads, S = STAGES: in phase 2j every wave issues its share of tile
    // j+S-1 into stage (j-1) % S (its previous tile, j-1, was read in phases 2j-2
    // and 2j-1), and at the end of phase 2j+1 waits until at most S-2 of its
    // tiles are in flight -- tile j+1 has landed -- so the barrier ending phase
    // 2j+1 publishes it.  Barriers per wave: 2 nk (phases 0 .. 2nk-1); group 1's
    // last MFMA phase (2nk) has none and runs while group 0 reaches the epilogue.
    // Group g = wave / 4: waves w and w + 4 share a SIMD whatever the 8-wave grid.
    // Each wave issues the tiles in order (group 1 one tile ahead of group 0), so
    // the conv loaders take the next tile from the issue cursor.
    static_assert(WM * WN == 8 && STAGES >= 2 && (EPI == EPI_STORE || EPI == EPI_LN_CR),
                  "ping-pong: 8 waves (one wave of each group per SIMD), a staged-store epilogue");
    // The fragments of one tile live from its memory phase to its MFMA phase of
    // the same iteration only; the accumulators are the only loop-carried state.
    auto read_tile = [&](auto J, int kt, Frag (&fa_)[NKS][G::TM], Frag (&fb_)[NKS][G::TN]) ICPP_INLINE {
      const char ICPP_LDS* as = stage_base(J);
      const int tap = tap_of(kt);
      static_for<NKS>([&](auto KS) ICPP_INLINE {
        constexpr int ks = decltype(KS)::value;
        load_frags(as, as + A_OFF, KS, fa_[ks], fb_[ks], tap);
      });
    };
    auto mfma_tile = [&](Frag (&fa_)[NKS][G::TM], Frag (&fb_)[NKS][G::TN]) ICPP_INLINE {
      static_for<NKS>([&](auto KS) ICPP_INLINE {
        constexpr int ks = decltype(KS)::value;
        mfma_step(fa_[ks], fb_[ks]);
      });
    };
    auto phase_end = [&]() ICPP_INLINE {
      __builtin_amdgcn_sched_barrier(0);
      lds_barrier();
      __builtin_amdgcn_sched_barrier(0);
    };
    // memory phase: the tile loads spread over the fragment reads
    auto sched_mem = [&]() ICPP_INLINE {
      constexpr int DS = NKS * DS_PER_KS;
      static_for<LOADS>([&](auto I) ICPP_INLINE {
        constexpr int i = decltype(I)::value;
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        constexpr int ds = (i + 1) * DS / LOADS - i * DS / LOADS;
        if constexpr (ds > 0) __builtin_amdgcn_sched_group_barrier(0x100, ds, 0);
      });
    };
    // MFMA phase: NL tile loads spread over the MFMAs
    auto sched_mfma = [&](auto NL) ICPP_INLINE {
      constexpr int nl = decltype(NL)::value;
      constexpr int NM = NKS * MFMA_PER_KS;
      static_for<NM>([&](auto I) ICPP_INLINE {
        constexpr int i = decltype(I)::value;
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        constexpr int l = (i + 1) * nl / NM - i * nl / NM;
        if constexpr (l > 0) __builtin_amdgcn_sched_group_barrier(0x020, l, 0);
      });
    };
    // K element of tile t; past the last tile the fetch is clamped to it (a cached
    // re-read into a stage nobody reads again), so every even phase issues LOADS loads
    const int kbase = first.kz * p.k_split;
    auto tile_k = [&](int t) ICPP_INLINE { return kbase + min(t, nk - 1) * BK; };
    auto tile_boff = [&](int t) ICPP_INLINE { return (uint32_t)(tile_k(t) * p.ldb * ESZ); };
    // issue tile t (this wave's next) into stage ST
    auto issue_seq = [&](auto ST, int t) ICPP_INLINE {
      if constexpr (DENSE) {
        issue_tile(tile_k(t), ST, TileCtx{0, 0}, tile_boff(t));
      } else {
        issue_tile(cur_kk(), ST, cursor_ctx(), cur_boff());
        advance_issue();
      }
    };
    constexpr int S = STAGES;
    static_for<S - 1>([&](auto I) ICPP_INLINE { issue_seq(I, decltype(I)::value); });
    wait_tiles(std::integral_constant<int, S - 2>{});  // this wave's loads of tile 0 landed
    lds_barrier();                                     // tile 0 published
    if (__builtin_amdgcn_readfirstlane(wave) < 4) {
      for (int kt0 = 0; kt0 < nk; kt0 += S) {
        static_for<S>([&](auto J) ICPP_INLINE {
          constexpr int j = decltype(J)::value;
          const int kt = kt0 + j;
          if (kt < nk) {
            Frag fa_[NKS][G::TM], fb_[NKS][G::TN];
            // phase 2kt: issue tile kt+S-1, read tile kt
            issue_seq(std::integral_constant<int, (j + S - 1) % S>{}, kt + S - 1);
            read_tile(J, kt, fa_, fb_);
            sched_mem();
            phase_end();
            // phase 2kt+1: multiply tile kt; then this wave's loads of tile kt+1 have landed
            mfma_tile(fa_, fb_);
            sched_mfma(std::integral_constant<int, 0>{});
            // a scheduling fence keeps the wait behind the MFMAs (left free, the
            // scheduler hoists it to the start of the phase and the MFMAs stall on
            // the loads just issued)
            __builtin_amdgcn_sched_barrier(0);
            wait_tiles(std::integral_constant<int, S - 2>{});
            phase_end();
          }
        });
      }
    } else {
      issue_seq(std::integral_constant<int, S - 1>{}, S - 1);
      phase_end();  // phase 0: group 1 has nothing to multiply yet
      for (int kt0 = 0; kt0 < nk; kt0 += S) {
        static_for<S>([&](auto J) ICPP_INLINE {
          constexpr int j = decltype(J)::value;
          const int kt = kt0 + j;
          if (kt < nk) {
            Frag fa_[NKS][G::TM], fb_[NKS][G::TN];
            // phase 2kt+1: read tile kt; this wave's loads of tile kt+1 have landed
            read_tile(J, kt, fa_, fb_);
            __builtin_amdgcn_sched_barrier(0);
            wait_tiles(std::integral_constant<int, S - 2>{});
            phase_end();
            // phase 2kt+2: multiply tile kt; issue tile kt+S into the stage tile kt leaves
            issue_seq(J, kt + S);
            mfma_tile(fa_, fb_);
            sched_mfma(std::integral_constant<int, LOADS>{});
            if (kt + 1 < nk) phase_end();
          }
        });
      }
    }
  } else {
  static_for<STAGES>([&](auto S) ICPP_INLINE {
    if constexpr (decltype(S)::value > 0) advance_issue();
    issue_tile(cur_kk(), S, cursor_ctx(), cur_boff());
  });
  wait_tiles(std::integral_constant<int, STAGES - 1>{});  // this wave's loads of tile 0 landed
  lds_barrier();  // tile 0 published
  load_frags(stage_base(std::integral_constant<int, 0>{}), stage_base(std::integral_constant<int, 0>{}) + A_OFF,
             std::integral_constant<int, 0>{}, fa[0], fb[0], tap_of(0));
  // One K tile in stage J: its NKS K-steps.
  auto tile_body = [&](auto J, int kt) ICPP_INLINE {
    constexpr int j = decltype(J)::value;
    const char ICPP_LDS* as = stage_base(J);
    static_for<NKS>([&](auto KS) ICPP_INLINE {
      constexpr int ks = decltype(KS)::value;
      constexpr int s = j * NKS + ks;  // position in the fragment double buffer
      if constexpr (ks + 1 < NKS) {
        load_frags(as, as + A_OFF, std::integral_constant<int, ks + 1>{}, fa[(s + 1) & 1], fb[(s + 1) & 1],
                   tap_of(kt));
        mfma_step(fa[s & 1], fb[s & 1]);
        schedule(std::integral_constant<int, 0>{});
      } else {
        advance_issue();                      // cursor -> step kt+STAGES (clamped)
        wait_tiles(std::integral_constant<int, STAGES - 2>{});  // this wave's loads of tile kt+1 landed
        lds_barrier();                        // B(kt): tile kt+1 published, stage j retired
        issue_tile(cur_kk(), J, cursor_ctx(), cur_boff());
        constexpr int jn = (j + 1) % STAGES;
        const char ICPP_LDS* an = stage_base(std::integral_constant<int, jn>{});
        load_frags(an, an + A_OFF, std::integral_constant<int, 0>{}, fa[(s + 1) & 1], fb[(s + 1) & 1],
                   tap_of(kt + 1));
        mfma_step(fa[s & 1], fb[s & 1]);
        schedule(std::integral_constant<int, LOADS>{});
      }
    });
  };
  // Whole rounds of STAGES tiles run unguarded, so a round is one basic block (the
  // stage of each tile is a compile-time constant: kt0 % STAGES == 0), and the
  // remaining nk % STAGES tiles follow, one guard each.  With a guard per tile in
  // the loop, the backend guarded the first fragment read of each tile's block
  // with a vmcnt(0) wait -- a stall on the tile loads just issued (1.5-3.5% on
  // 256x256 tiles).  The separate tail needs registers of its own, so tiles that
  // already hold 128 accumulators per lane keep the guarded loop (peeling them
  // spills); their ping-pong twins have no such wait.
  constexpr bool PEEL = (BM * BN) / (WM * WN * 64) < 128;
  if constexpr (PEEL) {
    const int nfull = nk - nk % STAGES;
    for (int kt0 = 0; kt0 < nfull; kt0 += STAGES)
      static_for<STAGES>([&](auto J) ICPP_INLINE { tile_body(J, kt0 + decltype(J)::value); });
    static_for<STAGES - 1>([&](auto J) ICPP_INLINE {
      if (nfull + decltype(J)::value < nk) tile_body(J, nfull + decltype(J)::value);
    });
  } else {
    for (int kt0 = 0; kt0 < nk; kt0 += STAGES)
      static_for<STAGES>([&](auto J) ICPP_INLINE {
        if (kt0 + decltype(J)::value < nk) tile_body(J, kt0 + decltype(J)::value);
      });
  }
  }
  wait_vmcnt<0>();  // no LDS-DMA write may land after this point (epilogue staging, next workgroup)
  epilogue(first);
}

// ---------------------------------------------------------------------------
// Split-K reduction + epilogue: C = act(alpha * sum_z ws[z] + bias)
// ---------------------------------------------------------------------------
// With ce.flags set (conv instances), the fused conv epilogue replaces bias/alpha.
template <int DT>
__global__ void __launch_bounds__(256)
splitk_reduce_kernel(const float* __restrict__ ws, void* C, const void* bias, int M, int N, int ldc,
                     int splits, float alpha, int act, ConvEpiArgs ce) {
  const size_t groups = (size_t)M * (N / 4);
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t gi = (size_t)blockIdx.x * blockDim.x + threadIdx.x; gi < groups; gi += stride)
    splitk_group<DT>(ws, C, bias, M, N, ldc, splits, alpha, act, ce, (int)(gi / (N / 4)), (int)(gi % (N / 4)) * 4);
}

// ---------------------------------------------------------------------------
// Two-pass LayerNorm finalize: combine per-(row, column block) (mean, M2)
// partials (Chan et al. pairwise update), then normalise the row in place.  The
// GEMM stored each block centred on its own mean, so x = stored + (block mean -
// row mean) relative to the row mean.  One wave per row; 4 rows per 256-thread
// workgroup.
// ---------------------------------------------------------------------------
template <int DT>
__global__ void __launch_bounds__(256)
ln_finalize_kernel(void* C, const float* __restrict__ stats, const void* gamma, const void* beta,
                   int M, int N, int ldc, int stat_cols, int block_cols, float eps) {
  typedef typename DTraits<DT>::OutT OutT;
  typedef typename DTraits<DT>::BiasT BiasT;
  const int lane = threadIdx.x & 63;
  const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (m >= M) return;
  // every lane combines all partials (stat_cols is small) so no broadcast is needed
  float n_acc = 0.f, mean = 0.f, m2 = 0.f;
  for (int j = 0; j < stat_cols; ++j) {
    const float nb = (float)max(0, min(block_cols, N - j * block_cols));
    if (nb <= 0.f) continue;
    const float mb = stats[((size_t)m * stat_cols + j) * 2 + 0];
    const float qb = stats[((size_t)m * stat_cols + j) * 2 + 1];
    const float nt = n_acc + nb;
    const float d = mb - mean;
    mean += d * (nb / nt);
    m2 += qb + d * d * (n_acc * nb / nt);
    n_acc = nt;
  }
  const float rstd = rsqrtf(m2 / (float)N + eps);
  OutT* row = (OutT*)C + (size_t)m * ldc;
  const BiasT* g = (const BiasT*)gamma;
  const BiasT* b = (const BiasT*)beta;
  for (int n = lane * 4; n < N; n += 256) {
    f32x4 x = Vec4Store<OutT>::ld(row + n);
    const f32x4 gv = Vec4Store<BiasT>::ld(g + n);
    const f32x4 bv = Vec4Store<BiasT>::ld(b + n);
    // block_cols is a multiple of 4, so the 4 columns share one block
    const float d = stats[((size_t)m * stat_cols + n / block_cols) * 2 + 0] - mean;
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] = (x[e] + d) * rstd * gv[e] + bv[e];
    Vec4Store<OutT>::st(row + n, x);
  }
}

}  // namespace icpp
