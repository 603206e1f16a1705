// Row-wise kernels for gfx950: LayerNorm forward / backward and softmax over the
// last dimension of a [M, N] row-major tensor (row stride ld >= N).
//
// Reference: kernel/triton/layernorm.py (_layer_norm_fwd_fused :48-91,
// _layer_norm_bwd_dx_fused :128-181, _layer_norm_bwd_dwdb :184-207,
// LayerNorm.forward/backward :219-275) and kernel/triton/softmax.py
// (softmax_kernel :32-55, softmax :73-102).
//
// Layout: each row is split into chunks of VEC elements (16 bytes: 8 x f16/bf16,
// 4 x f32; VEC = 1 when N, the strides or the pointers are not 16-byte multiples).
// TPR threads share a row (a power of two, 64..1024); thread t owns chunks
// t, t + TPR, ... (CPT of them), so each wave instruction reads a contiguous
// 1 KiB of the row. A row is loaded into registers once: every statistic and
// the output come from registers (HBM traffic = the algorithmic bytes).
// Reductions: xor-shuffles within the wave, then LDS across the row's waves.
//
// LayerNorm backward writes dx per row and accumulates dw / db in fp32
// registers: a persistent grid of G <= 256 workgroups walks the rows, each
// thread always owning the same columns; the row slots of a workgroup are
// folded together through LDS and one fp32 partial row per workgroup goes to
// the workspace, which a column-sum kernel reduces in a fixed order
// (deterministic; no locks or atomics, unlike the reference's
// lock-protected fp16 partial buffers).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "icpp_hip.h"

namespace icpp_rows {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int MAX_WAVES = 16;   // 1024 threads
constexpr int BWD_BLOCK = 1024;
constexpr int BWD_MAX_GROUPS = 256;

template <typename T> __device__ __forceinline__ float to_f(T v) { return (float)v; }
template <typename T> __device__ __forceinline__ T from_f(float v) { return (T)v; }

// VEC elements of T at p (16-byte aligned when VEC > 1) <-> floats
template <typename T, int VEC>
__device__ __forceinline__ void load_chunk(const T* p, float* out) {
  if constexpr (VEC == 1) {
    out[0] = to_f(*p);
  } else {
    const i32x4 raw = *reinterpret_cast<const i32x4*>(p);
    T e[VEC];
    __builtin_memcpy(e, &raw, 16);
#pragma unroll
    for (int i = 0; i < VEC; ++i) out[i] = to_f(e[i]);
  }
}
template <typename T, int VEC>
__device__ __forceinline__ void store_chunk(T* p, const float* in) {
  if constexpr (VEC == 1) {
    *p = from_f<T>(in[0]);
  } else {
    T e[VEC];
#pragma unroll
    for (int i = 0; i < VEC; ++i) e[i] = from_f<T>(in[i]);
    i32x4 raw;
    __builtin_memcpy(&raw, e, 16);
    __builtin_nontemporal_store(raw, reinterpret_cast<i32x4*>(p));
  }
}

struct Sum { __device__ float operator()(float a, float b) const { return a + b; } };
struct Max { __device__ float operator()(float a, float b) const { return fmaxf(a, b); } };

template <typename Op>
__device__ __forceinline__ float wave_reduce(float v, Op op) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = op(v, __shfl_xor(v, off, 64));
  return v;
}

// Reduce v over the TPR threads of each row. Every thread of the block calls it
// the same number of times (one __syncthreads each); slot alternates between two
// LDS buffers so a reduction never overwrites values another wave may still read.
template <typename Op>
__device__ __forceinline__ float row_reduce(float v, Op op, int tpr, float (*red)[MAX_WAVES], int& slot) {
  v = wave_reduce(v, op);
  if (tpr <= 64) return v;
  const int wave = threadIdx.x >> 6;
  const int wpr = tpr >> 6;                // waves per row
  const int first = (wave / wpr) * wpr;    // first wave of this row
  if ((threadIdx.x & 63) == 0) red[slot][wave] = v;
  __syncthreads();
  float r = red[slot][first];
  for (int w = 1; w < wpr; ++w) r = op(r, red[slot][first + w]);
  slot ^= 1;
  return r;
}

// Two row sums behind one workgroup barrier, each summed in row_reduce's order.
// The two pair buffers alternate like row_reduce's slots: the next pair's writes
// cannot overtake a slow wave still reading this one, because the barrier of the
// pair in between lies between them.
__device__ __forceinline__ void row_reduce2(float& a, float& b, int tpr, float (*red)[2][MAX_WAVES], int& slot) {
  a = wave_reduce(a, Sum{});
  b = wave_reduce(b, Sum{});
  if (tpr <= 64) return;
  const int wave = threadIdx.x >> 6;
  const int wpr = tpr >> 6;                // waves per row
  const int first = (wave / wpr) * wpr;    // first wave of this row
  if ((threadIdx.x & 63) == 0) {
    red[slot][0][wave] = a;
    red[slot][1][wave] = b;
  }
  __syncthreads();
  float ra = red[slot][0][first], rb = red[slot][1][first];
  for (int w = 1; w < wpr; ++w) {
    ra += red[slot][0][first + w];
    rb += red[slot][1][first + w];
  }
  slot ^= 1;
  a = ra;
  b = rb;
}

// ---------------------------------------------------------------------------
// LayerNorm forward: y = (x - mean) * rstd * w + b, mean / rstd (fp32) per row
// (reference _layer_norm_fwd_fused: centred two-pass variance, rstd = 1/sqrt(var+eps)).
// ---------------------------------------------------------------------------
// With a residual R (may be null), x = X + R (R has X's row stride).  With block
// means BMN (may be null; [M][bm_cols] fp32, block j covering columns
// j*bm_width .. +bm_width-1, bm_width a multiple of VEC) x also gains its block's
// mean: X then holds values stored centred on those means by the producing GEMM.
// Y may be X: every row is held in registers before any of it is written.
template <typename T, int VEC, int CPT>
__global__ void __launch_bounds__(1024)
layernorm_fwd_kernel(const T* X, const T* R, const float* __restrict__ BMN, const T* __restrict__ W,
                     const T* __restrict__ B, T* Y, float* __restrict__ mean_out, float* __restrict__ rstd_out, int M,
                     int N, int ldx, int ldy, float eps, int tpr, int bm_cols, int bm_width) {
  __shared__ float red[2][MAX_WAVES];
  int slot = 0;
  const int rpb = blockDim.x / tpr;
  const int row = blockIdx.x * rpb + threadIdx.x / tpr;
  const int t = threadIdx.x % tpr;
  const bool live = row < M;
  const int nch = (N + VEC - 1) / VEC;
  float x[CPT][VEC];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = t + i * tpr;
    if (live && c < nch) {
      load_chunk<T, VEC>(X + (size_t)row * ldx + (size_t)c * VEC, x[i]);
      if (R != nullptr) {
        float r[VEC];
        load_chunk<T, VEC>(R + (size_t)row * ldx + (size_t)c * VEC, r);
#pragma unroll
        for (int e = 0; e < VEC; ++e) x[i][e] += r[e];
      }
      if (BMN != nullptr) {
        const float bm = BMN[(size_t)row * bm_cols + (c * VEC) / bm_width];
#pragma unroll
        for (int e = 0; e < VEC; ++e) x[i][e] += bm;
      }
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) x[i][e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) s += x[i][e];
  }
  const float mean = row_reduce(s, Sum{}, tpr, red, slot) / (float)N;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = t + i * tpr;
    if (c < nch) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float d = x[i][e] - mean;
        q += d * d;
      }
    }
  }
  const float var = row_reduce(q, Sum{}, tpr, red, slot) / (float)N;
  const float rstd = 1.f / sqrtf(var + eps);
  if (live && t == 0) {
    if (mean_out) mean_out[row] = mean;
    if (rstd_out) rstd_out[row] = rstd;
  }
  if (!live) return;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = t + i * tpr;
    if (c < nch) {
      float w[VEC], b[VEC], y[VEC];
      load_chunk<T, VEC>(W + (size_t)c * VEC, w);
      load_chunk<T, VEC>(B + (size_t)c * VEC, b);
#pragma unroll
      for (int e = 0; e < VEC; ++e) y[e] = (x[i][e] - mean) * rstd * w[e] + b[e];
      store_chunk<T, VEC>(Y + (size_t)row * ldy + (size_t)c * VEC, y);
    }
  }
}

// ---------------------------------------------------------------------------
// Softmax over each row: exp(x - max) / sum (reference softmax_kernel; the
// arithmetic is fp32 whatever the storage type).  SCALED: the row is first
// x * scale + mask[row % mask_rows] (mask [mask_rows, N], row stride N, or null):
// the attention scores of the BERT layer (end2end.py:52-66: q k^T / sqrt(d) +
// causal mask, then softmax) in one pass.
// ---------------------------------------------------------------------------
template <typename T, int VEC, int CPT, bool SCALED>
__global__ void __launch_bounds__(1024)
softmax_kernel(const T* __restrict__ X, T* __restrict__ Y, int M, int N, int ldx, int ldy, int tpr,
               const T* __restrict__ mask, float scale, int mask_rows) {
  __shared__ float red[2][MAX_WAVES];
  int slot = 0;
  const int rpb = blockDim.x / tpr;
  const int row = blockIdx.x * rpb + threadIdx.x / tpr;
  const int t = threadIdx.x % tpr;
  const bool live = row < M;
  const int nch = (N + VEC - 1) / VEC;
  float x[CPT][VEC];
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = t + i * tpr;
    if (live && c < nch) {
      load_chunk<T, VEC>(X + (size_t)row * ldx + (size_t)c * VEC, x[i]);
      if constexpr (SCALED) {
        float mk[VEC];
        if (mask != nullptr) load_chunk<T, VEC>(mask + (size_t)(row % mask_rows) * N + (size_t)c * VEC, mk);
#pragma unroll
        for (int e = 0; e < VEC; ++e) x[i][e] = x[i][e] * scale + (mask != nullptr ? mk[e] : 0.f);
      }
#pragma unroll
      for (int e = 0; e < VEC; ++e) m = fmaxf(m, x[i][e]);
    }
  }
  m = row_reduce(m, Max{}, tpr, red, slot);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = t + i * tpr;
    if (live && c < nch) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        x[i][e] = expf(x[i][e] - m);
        s += x[i][e];
      }
    }
  }
  s = row_reduce(s, Sum{}, tpr, red, slot);
  if (!live) return;
  const float inv = 1.f / s;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = t + i * tpr;
    if (c < nch) {
      float y[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) y[e] = x[i][e] * inv;
      store_chunk<T, VEC>(Y + (size_t)row * ldy + (size_t)c * VEC, y);
    }
  }
}

// ---------------------------------------------------------------------------
// LayerNorm backward, pass 1 (reference _layer_norm_bwd_dx_fused :128-181):
//   xhat = (x - mean) * rstd, wdy = w * dy
//   c1 = sum(xhat * wdy) / N, c2 = sum(wdy) / N
//   dx = (wdy - (xhat * c1 + c2)) * rstd
// plus dw = sum_rows dy * xhat and db = sum_rows dy, accumulated per thread in
// fp32 and written as one partial row per workgroup: part[g][0..N) = dw,
// part[g][N..2N) = db.
// ---------------------------------------------------------------------------
// One row chunk as stored: 16 bytes (VEC elements), or a single element.
template <typename T, int VEC>
struct Chunk {
  typedef i32x4 raw;
  static __device__ __forceinline__ raw load(const T* p) { return *reinterpret_cast<const i32x4*>(p); }
  static __device__ __forceinline__ raw zero() { return i32x4{0, 0, 0, 0}; }
  static __device__ __forceinline__ void unpack(const raw& r, float* out) {
    T e[VEC];
    __builtin_memcpy(e, &r, 16);
#pragma unroll
    for (int i = 0; i < VEC; ++i) out[i] = to_f(e[i]);
  }
};
template <typename T>
struct Chunk<T, 1> {
  typedef T raw;
  static __device__ __forceinline__ raw load(const T* p) { return *p; }
  static __device__ __forceinline__ raw zero() { return from_f<T>(0.f); }
  static __device__ __forceinline__ void unpack(const raw& r, float* out) { out[0] = to_f(r); }
};

template <typename T, int VEC, int CPT>
__global__ void __launch_bounds__(BWD_BLOCK)
layernorm_bwd_kernel(const T* __restrict__ DY, const T* __restrict__ X, const T* __restrict__ W,
                     const float* __restrict__ mean_in, const float* __restrict__ rstd_in, T* __restrict__ DX,
                     float* __restrict__ part, int M, int N, int ld, int tpr) {
  typedef Chunk<T, VEC> Ch;
  typedef typename Ch::raw Raw;
  __shared__ float red[2][2][MAX_WAVES];
  __shared__ f32x4 fold[BWD_BLOCK];  // row-slot folding, one 16-byte value per thread
  int slot = 0;
  const int rpb = blockDim.x / tpr;
  const int rs = threadIdx.x / tpr;  // row slot within the workgroup
  const int t = threadIdx.x % tpr;
  const int nch = (N + VEC - 1) / VEC;
  const float inv_n = 1.f / (float)N;
  // x, dy and w stay in their storage type (half the registers of fp32 copies for
  // 16-bit data), so the next rows' chunks can be in flight while this row reduces
  Raw wr[CPT];
  float dw[CPT][VEC], db[CPT][VEC];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = t + i * tpr;
    wr[i] = c < nch ? Ch::load(W + (size_t)c * VEC) : Ch::zero();
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      dw[i][e] = 0.f;
      db[i][e] = 0.f;
    }
  }
  static_assert((int)sizeof(T) * VEC * CPT <= 16, "prefetching backward: at most 16 bytes of a row per thread");
  Raw nx[CPT], ndy[CPT];
  float nmean = 0.f, nrstd = 0.f;
  auto fetch = [&](int row) {
    const bool live = row < M;
    nmean = live ? mean_in[row] : 0.f;
    nrstd = live ? rstd_in[row] : 0.f;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = t + i * tpr;
      const bool ok = live && c < nch;
      nx[i] = ok ? Ch::load(X + (size_t)row * ld + (size_t)c * VEC) : Ch::zero();
      ndy[i] = ok ? Ch::load(DY + (size_t)row * ld + (size_t)c * VEC) : Ch::zero();
    }
  };
  // rows rs + rpb * (blockIdx.x + k * gridDim.x): every thread runs the same trip count
  const int stride = rpb * gridDim.x;
  fetch(blockIdx.x * rpb + rs);
  for (int base = blockIdx.x * rpb; base < M; base += stride) {
    const int row = base + rs;
    const bool live = row < M;
    Raw cx[CPT], cdy[CPT];
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      cx[i] = nx[i];
      cdy[i] = ndy[i];
    }
    const float mean = nmean, rstd = nrstd;
    if (base + stride < M) fetch(base + stride + rs);  // the next rows load during this row's reductions
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = t + i * tpr;
      float xv[VEC], dyv[VEC], w[VEC];
      Ch::unpack(cx[i], xv);
      Ch::unpack(cdy[i], dyv);
      Ch::unpack(wr[i], w);
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float xh = (live && c < nch) ? (xv[e] - mean) * rstd : 0.f;
        const float wdy = w[e] * dyv[e];
        s1 += xh * wdy;
        s2 += wdy;
      }
    }
    row_reduce2(s1, s2, tpr, red, slot);
    const float c1 = s1 * inv_n;
    const float c2 = s2 * inv_n;
    if (live) {
#pragma unroll
      for (int i = 0; i < CPT; ++i) {
        const int c = t + i * tpr;
        if (c < nch) {
          float xv[VEC], dyv[VEC], w[VEC], dx[VEC];
          Ch::unpack(cx[i], xv);
          Ch::unpack(cdy[i], dyv);
          Ch::unpack(wr[i], w);
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            const float xh = (xv[e] - mean) * rstd;
            const float wdy = w[e] * dyv[e];
            dx[e] = (wdy - (xh * c1 + c2)) * rstd;
            dw[i][e] += dyv[e] * xh;
            db[i][e] += dyv[e];
          }
          store_chunk<T, VEC>(DX + (size_t)row * ld + (size_t)c * VEC, dx);
        }
      }
    }
  }
  // fold the row slots into slot 0 (fixed order: slot 0 + 1 + 2 + ...), 4 floats at a time
  float* out = part + (size_t)blockIdx.x * 2 * N;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
#pragma unroll
    for (int which = 0; which < 2; ++which) {
#pragma unroll
      for (int e0 = 0; e0 < VEC; e0 += 4) {
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (e0 + e < VEC) ? (which ? db[i][e0 + e] : dw[i][e0 + e]) : 0.f;
        __syncthreads();  // previous round's reads are done
        fold[threadIdx.x] = v;
        __syncthreads();
        if (rs == 0) {
          for (int r = 1; r < rpb; ++r) v += fold[r * tpr + t];
          const int c = t + i * tpr;
          if (c < nch) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (e0 + e < VEC) out[(size_t)which * N + (size_t)c * VEC + e0 + e] = v[e];
          }
        }
      }
    }
  }
}

// Rows longer than one 16-byte chunk per thread (2 chunks, N <= 16384 for 16-bit
// types): x, dy, xhat and w*dy of the row in fp32 registers, no prefetch.
template <typename T, int VEC, int CPT>
__global__ void __launch_bounds__(BWD_BLOCK)
layernorm_bwd_kernel_long(const T* __restrict__ DY, const T* __restrict__ X, const T* __restrict__ W,
                     const float* __restrict__ mean_in, const float* __restrict__ rstd_in, T* __restrict__ DX,
                     float* __restrict__ part, int M, int N, int ld, int tpr) {
  __shared__ float red[2][2][MAX_WAVES];
  __shared__ f32x4 fold[BWD_BLOCK];  // row-slot folding, one 16-byte value per thread
  int slot = 0;
  const int rpb = blockDim.x / tpr;
  const int rs = threadIdx.x / tpr;  // row slot within the workgroup
  const int t = threadIdx.x % tpr;
  const int nch = (N + VEC - 1) / VEC;
  const float inv_n = 1.f / (float)N;
  float w[CPT][VEC], dw[CPT][VEC], db[CPT][VEC];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = t + i * tpr;
    if (c < nch) load_chunk<T, VEC>(W + (size_t)c * VEC, w[i]);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      if (c >= nch) w[i][e] = 0.f;
      dw[i][e] = 0.f;
      db[i][e] = 0.f;
    }
  }
  // rows rs + rpb * (blockIdx.x + k * gridDim.x): every thread runs the same trip count
  const int stride = rpb * gridDim.x;
  for (int base = blockIdx.x * rpb; base < M; base += stride) {
    const int row = base + rs;
    const bool live = row < M;
    const float mean = live ? mean_in[row] : 0.f;
    const float rstd = live ? rstd_in[row] : 0.f;
    float xh[CPT][VEC], wdy[CPT][VEC], dyv[CPT][VEC];
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = t + i * tpr;
      float xv[VEC];
      if (live && c < nch) {
        load_chunk<T, VEC>(X + (size_t)row * ld + (size_t)c * VEC, xv);
        load_chunk<T, VEC>(DY + (size_t)row * ld + (size_t)c * VEC, dyv[i]);
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) { xv[e] = 0.f; dyv[i][e] = 0.f; }
      }
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        xh[i][e] = (live && c < nch) ? (xv[e] - mean) * rstd : 0.f;
        wdy[i][e] = w[i][e] * dyv[i][e];
        s1 += xh[i][e] * wdy[i][e];
        s2 += wdy[i][e];
      }
    }
    row_reduce2(s1, s2, tpr, red, slot);
    const float c1 = s1 * inv_n;
    const float c2 = s2 * inv_n;
    if (live) {
#pragma unroll
      for (int i = 0; i < CPT; ++i) {
        const int c = t + i * tpr;
        if (c < nch) {
          float dx[VEC];
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            dx[e] = (wdy[i][e] - (xh[i][e] * c1 + c2)) * rstd;
            dw[i][e] += dyv[i][e] * xh[i][e];
            db[i][e] += dyv[i][e];
          }
          store_chunk<T, VEC>(DX + (size_t)row * ld + (size_t)c * VEC, dx);
        }
      }
    }
  }
  // fold the row slots into slot 0 (fixed order: slot 0 + 1 + 2 + ...), 4 floats at a time
  float* out = part + (size_t)blockIdx.x * 2 * N;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
#pragma unroll
    for (int which = 0; which < 2; ++which) {
#pragma unroll
      for (int e0 = 0; e0 < VEC; e0 += 4) {
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (e0 + e < VEC) ? (which ? db[i][e0 + e] : dw[i][e0 + e]) : 0.f;
        __syncthreads();  // previous round's reads are done
        fold[threadIdx.x] = v;
        __syncthreads();
        if (rs == 0) {
          for (int r = 1; r < rpb; ++r) v += fold[r * tpr + t];
          const int c = t + i * tpr;
          if (c < nch) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (e0 + e < VEC) out[(size_t)which * N + (size_t)c * VEC + e0 + e] = v[e];
          }
        }
      }
    }
  }
}

// Pass 2 (reference _layer_norm_bwd_dwdb :184-207): dw[n] = sum_g part[g][n],
// db[n] = sum_g part[g][N + n], summed in a fixed order. Workgroup of 256 = 32
// columns x 8 partial-row lanes, so a wave reads two whole 128-byte row segments
// per load; lane l sums partial rows l, l + 8, ... (G <= 256: at most 32, all
// issued before the first add), then the 8 lane sums are added in lane order
// through LDS.
constexpr int DWDB_COLS = 32, DWDB_LANES = 8;
template <typename T>
__global__ void __launch_bounds__(256)
layernorm_dwdb_kernel(const float* __restrict__ part, T* __restrict__ DW, T* __restrict__ DB, int G, int N) {
  __shared__ float acc[DWDB_LANES][DWDB_COLS + 1];
  const int col = threadIdx.x % DWDB_COLS, lane_g = threadIdx.x / DWDB_COLS;
  const int n2 = blockIdx.x * DWDB_COLS + col;  // column of the [dw | db] row of length 2N
  constexpr int PER = BWD_MAX_GROUPS / DWDB_LANES;  // partial rows per lane
  float v[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int g = lane_g + DWDB_LANES * j;
    v[j] = (n2 < 2 * N && g < G) ? part[(size_t)g * 2 * N + n2] : 0.f;
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < PER; ++j) s += v[j];
  acc[lane_g][col] = s;
  __syncthreads();
  if (lane_g == 0 && n2 < 2 * N) {
    float t = acc[0][col];
    for (int l = 1; l < DWDB_LANES; ++l) t += acc[l][col];
    if (n2 < N) DW[n2] = from_f<T>(t);
    else DB[n2 - N] = from_f<T>(t);
  }
}

// ---------------------------------------------------------------------------
// Attention head layout (BERT attention core, head_dim 64)
// ---------------------------------------------------------------------------
// qkv_split_heads: the fused QKV projection [T = batch*seq, 3*H] (H = heads*64) plus
// its bias [3H] -> Q [batch, heads, seq, 64] and K, V per head, one of them
// transposed: TP = 1 gives K^T [batch, heads, 64, seq] and V [.., seq, 64] (the
// batched-product attention), TP = 2 gives K [.., seq, 64] and V^T [.., 64, seq]
// (the fused attention kernel).  A workgroup takes 64 rows of one (batch, head): it
// reads three 64 x 64 blocks (one 128-byte row segment per token), adds the bias
// in fp32 and rounds once (as torch's add of two 16-bit tensors), writes the
// untransposed parts as contiguous 8 KiB blocks and part TP through a padded LDS
// tile (row stride 66 elements, so a column read spreads over the banks) as 64
// rows of 64 tokens.  Every access is a 16-byte chunk; rows past seq are neither
// read nor written.
constexpr int HD = 64;            // head_dim this kernel serves
constexpr int KT_LD = HD + 2;     // LDS tile row stride (elements)
template <typename T, int TP>
__global__ void __launch_bounds__(256)
qkv_split_heads_kernel(const T* __restrict__ QKV, const T* __restrict__ bias, T* __restrict__ Q,
                       T* __restrict__ K, T* __restrict__ V, int seq, int heads) {
  __shared__ T kt[HD][KT_LD];
  const int s0 = blockIdx.x * HD, hh = blockIdx.y, bb = blockIdx.z;
  const int H = heads * HD;
  const size_t bh = (size_t)bb * heads + hh;
  // chunk q = tid + 256 * i of the 64 x 8 block: token row q / 8, 8-element chunk q % 8
#pragma unroll
  for (int part = 0; part < 3; ++part) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int q = threadIdx.x + 256 * i;
      const int r = q >> 3, c = q & 7;
      const int ss = s0 + r;
      if (ss >= seq) continue;
      const int col = part * H + hh * HD + c * 8;
      float v[8];
      load_chunk<T, 8>(QKV + ((size_t)bb * seq + ss) * (3 * (size_t)H) + col, v);
      if (bias != nullptr) {
        float bv[8];
        load_chunk<T, 8>(bias + col, bv);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] += bv[e];
      }
      if (part == TP) {
#pragma unroll
        for (int e = 0; e < 8; ++e) kt[c * 8 + e][r] = from_f<T>(v[e]);
      } else {
        store_chunk<T, 8>((part == 0 ? Q : part == 1 ? K : V) + (bh * seq + ss) * HD + c * 8, v);
      }
    }
  }
  __syncthreads();
  // rows of the transposed part: head dim d, 64 tokens s0 .. s0+63 (8 chunks of 8 tokens)
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int q = threadIdx.x + 256 * i;
    const int d = q >> 3, c = q & 7;
    const int ss = s0 + c * 8;
    if (ss >= seq) continue;
    T* out = (TP == 1 ? K : V) + (bh * HD + d) * (size_t)seq + ss;
    if (ss + 8 <= seq && (seq & 7) == 0) {
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = to_f(kt[d][c * 8 + e]);
      store_chunk<T, 8>(out, v);
    } else {
      for (int e = 0; e < 8 && ss + e < seq; ++e) out[e] = kt[d][c * 8 + e];
    }
  }
}

// merge_heads: context [batch, heads, seq, 64] -> [batch*seq, heads*64], one 16-byte
// chunk per lane, consecutive lanes on consecutive chunks of an output row.
template <typename T>
__global__ void __launch_bounds__(256)
merge_heads_kernel(const T* __restrict__ X, T* __restrict__ Y, int batch, int seq, int heads) {
  const size_t chunks = (size_t)batch * seq * heads * (HD / 8);
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x; q < chunks; q += stride) {
    const int c = (int)(q % (HD / 8));
    const size_t rest = q / (HD / 8);
    const int hh = (int)(rest % heads);
    const size_t t = rest / heads;  // token row bb * seq + ss
    const size_t bb = t / seq, ss = t % seq;
    const i32x4 v = *reinterpret_cast<const i32x4*>(X + ((bb * heads + hh) * seq + ss) * HD + c * 8);
    __builtin_nontemporal_store(v, reinterpret_cast<i32x4*>(Y + t * ((size_t)heads * HD) + hh * HD + c * 8));
  }
}

}  // namespace icpp_rows

// ---------------------------------------------------------------------------
// Host side: geometry choice, validation, dispatch
// ---------------------------------------------------------------------------
namespace icpp {
int set_last_error(int code, const char* msg);  // icpp_abi.hip: the library's last-error buffer
}

namespace {

using namespace icpp_rows;

int set_error(int code, const char* msg) { return icpp::set_last_error(code, msg); }

struct RowGeom {
  int vec, tpr, cpt, block;
};

int next_pow2(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}
bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
int esize(int dtype) { return dtype == ICPP_F32 ? 4 : 2; }

// Pick the chunk width, threads per row and chunks per thread for N columns.
// Returns false when N needs more than cpt_max chunks for each of 1024 threads.
bool row_geom(int N, int vec, int cpt_max, RowGeom* g) {
  const int nch = (N + vec - 1) / vec;
  int tpr = next_pow2((nch + cpt_max - 1) / cpt_max);
  tpr = tpr < 64 ? 64 : tpr;
  if (tpr > 1024) return false;
  g->vec = vec;
  g->tpr = tpr;
  g->cpt = next_pow2((nch + tpr - 1) / tpr);
  g->block = tpr >= 256 ? tpr : 256;
  return true;
}

template <typename T, typename F>
hipError_t dispatch_cpt(const RowGeom& g, F&& launch) {
  // VEC = 16 / sizeof(T) or 1; CPT 1..16 (the geometry keeps CPT within the kernel's limits)
  constexpr int V = 16 / (int)sizeof(T);
  if (g.vec == V) {
    switch (g.cpt) {
      case 1: return launch(std::integral_constant<int, V>{}, std::integral_constant<int, 1>{});
      case 2: return launch(std::integral_constant<int, V>{}, std::integral_constant<int, 2>{});
      case 4: return launch(std::integral_constant<int, V>{}, std::integral_constant<int, 4>{});
      default: return launch(std::integral_constant<int, V>{}, std::integral_constant<int, 8>{});
    }
  }
  switch (g.cpt) {
    case 1: return launch(std::integral_constant<int, 1>{}, std::integral_constant<int, 1>{});
    case 2: return launch(std::integral_constant<int, 1>{}, std::integral_constant<int, 2>{});
    case 4: return launch(std::integral_constant<int, 1>{}, std::integral_constant<int, 4>{});
    case 8: return launch(std::integral_constant<int, 1>{}, std::integral_constant<int, 8>{});
    default: return launch(std::integral_constant<int, 1>{}, std::integral_constant<int, 16>{});
  }
}

template <typename T>
int ln_fwd_t(const void* X, const void* R, const void* W, const void* B, void* Y, float* mean, float* rstd, int M,
             int N, int ldx, int ldy, float eps, hipStream_t s, const float* bmn = nullptr, int bm_cols = 0,
             int bm_width = 1) {
  constexpr int V = 16 / (int)sizeof(T);
  const bool vec_ok = N % V == 0 && ldx % V == 0 && ldy % V == 0 && aligned16(X) && aligned16(Y) &&
                      aligned16(W) && aligned16(B) && (R == nullptr || aligned16(R)) &&
                      (bmn == nullptr || bm_width % V == 0);
  RowGeom g;
  if (!row_geom(N, vec_ok ? V : 1, vec_ok ? 8 : 16, &g)) return set_error(ICPP_E_SHAPE, "icpp_layernorm_fwd: N too large");
  const int rpb = g.block / g.tpr;
  const dim3 grid((M + rpb - 1) / rpb);
  hipError_t e = dispatch_cpt<T>(g, [&](auto VEC, auto CPT) {
    hipLaunchKernelGGL((layernorm_fwd_kernel<T, decltype(VEC)::value, decltype(CPT)::value>), grid, dim3(g.block), 0, s,
                       (const T*)X, (const T*)R, bmn, (const T*)W, (const T*)B, (T*)Y, mean, rstd, M, N, ldx, ldy,
                       eps, g.tpr, bm_cols, bm_width);
    return hipGetLastError();
  });
  return e == hipSuccess ? ICPP_OK : set_error((int)e, hipGetErrorString(e));
}

template <typename T>
int softmax_t(const void* X, void* Y, int M, int N, int ldx, int ldy, hipStream_t s, bool scaled = false,
              const void* mask = nullptr, float scale = 1.f, int mask_rows = 1) {
  constexpr int V = 16 / (int)sizeof(T);
  const bool vec_ok = N % V == 0 && ldx % V == 0 && ldy % V == 0 && aligned16(X) && aligned16(Y) &&
                      (mask == nullptr || aligned16(mask));
  RowGeom g;
  if (!row_geom(N, vec_ok ? V : 1, vec_ok ? 8 : 16, &g)) return set_error(ICPP_E_SHAPE, "icpp_softmax: N too large");
  const int rpb = g.block / g.tpr;
  const dim3 grid((M + rpb - 1) / rpb);
  hipError_t e = dispatch_cpt<T>(g, [&](auto VEC, auto CPT) {
    constexpr int Vv = decltype(VEC)::value, Cc = decltype(CPT)::value;
    if (scaled)
      hipLaunchKernelGGL((softmax_kernel<T, Vv, Cc, true>), grid, dim3(g.block), 0, s, (const T*)X, (T*)Y, M, N, ldx,
                         ldy, g.tpr, (const T*)mask, scale, mask_rows);
    else
      hipLaunchKernelGGL((softmax_kernel<T, Vv, Cc, false>), grid, dim3(g.block), 0, s, (const T*)X, (T*)Y, M, N, ldx,
                         ldy, g.tpr, (const T*)nullptr, 1.f, 1);
    return hipGetLastError();
  });
  return e == hipSuccess ? ICPP_OK : set_error((int)e, hipGetErrorString(e));
}

// Backward geometry: w, dw, db and the row's x / dy stay in registers, and a
// 1024-thread workgroup leaves each wave 128 VGPRs.  One 16-byte chunk per
// thread (up to 1024 threads per row: N <= 8192 for 16-bit types) leaves room to
// prefetch the next rows; longer rows take 2 chunks per thread (N <= 16384)
// without the prefetch.  The scalar path holds at most 4 elements per thread.
bool bwd_geom(int dtype, int N, int ld, bool ptrs_aligned, RowGeom* g) {
  const int V = 16 / esize(dtype);
  const bool vec_ok = N % V == 0 && ld % V == 0 && ptrs_aligned;
  if (vec_ok ? !row_geom(N, V, 1, g) && !row_geom(N, V, 2, g) : !row_geom(N, 1, 4, g)) return false;
  g->block = BWD_BLOCK;
  return true;
}

int bwd_groups(int M, const RowGeom& g) {
  const int rpb = g.block / g.tpr;
  const int need = (M + rpb - 1) / rpb;
  return need < BWD_MAX_GROUPS ? need : BWD_MAX_GROUPS;
}

template <typename T>
int ln_bwd_t(const void* DY, const void* X, const void* W, const float* mean, const float* rstd, void* DX, void* DW,
             void* DB, int M, int N, int ld, const RowGeom& g, float* part, hipStream_t s) {
  const int G = bwd_groups(M, g);
  hipError_t e = dispatch_cpt<T>(g, [&](auto VEC, auto CPT) {
    if constexpr (decltype(CPT)::value > 4 || (decltype(VEC)::value > 1 && decltype(CPT)::value > 2)) {
      return hipErrorInvalidValue;  // outside the backward's register budget (row_geom never picks it)
    } else {
      constexpr int V = decltype(VEC)::value, C = decltype(CPT)::value;
      if constexpr ((int)sizeof(T) * V * C <= 16)
        hipLaunchKernelGGL((layernorm_bwd_kernel<T, V, C>), dim3(G), dim3(g.block), 0, s, (const T*)DY, (const T*)X,
                           (const T*)W, mean, rstd, (T*)DX, part, M, N, ld, g.tpr);
      else
        hipLaunchKernelGGL((layernorm_bwd_kernel_long<T, V, C>), dim3(G), dim3(g.block), 0, s, (const T*)DY,
                           (const T*)X, (const T*)W, mean, rstd, (T*)DX, part, M, N, ld, g.tpr);
      return hipGetLastError();
    }
  });
  if (e != hipSuccess) return set_error((int)e, hipGetErrorString(e));
  hipLaunchKernelGGL(layernorm_dwdb_kernel<T>, dim3((2 * N + DWDB_COLS - 1) / DWDB_COLS), dim3(256), 0, s, part, (T*)DW,
                     (T*)DB, G, N);
  e = hipGetLastError();
  return e == hipSuccess ? ICPP_OK : set_error((int)e, hipGetErrorString(e));
}

int check_rows(const char* fn, int dtype, int M, int N, int ld_in, int ld_out) {
  if (dtype != ICPP_F16 && dtype != ICPP_BF16 && dtype != ICPP_F32)
    return set_error(ICPP_E_ARG, fn);
  if (M <= 0 || N <= 0 || ld_in < N || ld_out < N) return set_error(ICPP_E_SHAPE, fn);
  if ((long long)M * ld_in > 0x7FFFFFFFll * 8 || (long long)M * ld_out > 0x7FFFFFFFll * 8)
    return set_error(ICPP_E_SHAPE, fn);
  return ICPP_OK;
}

}  // namespace

namespace icpp {
// Y = LayerNorm(X [+ R] + block_mean) * W + B over rows of an f16 [M, N] tensor (row
// stride N), Y may be X; for icpp_gemm_bias_residual_layernorm's GEMM-then-LayerNorm
// strategy, whose GEMM stores X centred on per-(row, bm_width-column block) means
// block_mean [M][bm_cols] (null: X is stored as is).
int layernorm_rows_f16(const void* X, const void* R, const float* block_mean, int bm_cols, int bm_width, const void* W,
                       const void* B, void* Y, int M, int N, float eps, hipStream_t s) {
  return ln_fwd_t<_Float16>(X, R, W, B, Y, nullptr, nullptr, M, N, N, N, eps, s, block_mean, bm_cols, bm_width);
}
}  // namespace icpp

extern "C" {

int icpp_layernorm_fwd(int dtype, const void* X, const void* W, const void* B, void* Y, float* mean, float* rstd,
                       int M, int N, int ldx, int ldy, float eps, void* stream) {
  if (!X || !W || !B || !Y) return set_error(ICPP_E_ARG, "icpp_layernorm_fwd: null tensor");
  if (int rc = check_rows("icpp_layernorm_fwd: bad dtype or shape", dtype, M, N, ldx, ldy)) return rc;
  if (!(eps >= 0.f)) return set_error(ICPP_E_ARG, "icpp_layernorm_fwd: eps must be >= 0");
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ICPP_F16) return ln_fwd_t<_Float16>(X, nullptr, W, B, Y, mean, rstd, M, N, ldx, ldy, eps, s);
  if (dtype == ICPP_BF16) return ln_fwd_t<__bf16>(X, nullptr, W, B, Y, mean, rstd, M, N, ldx, ldy, eps, s);
  return ln_fwd_t<float>(X, nullptr, W, B, Y, mean, rstd, M, N, ldx, ldy, eps, s);
}

size_t icpp_layernorm_bwd_workspace_bytes(int dtype, int M, int N, int ld) {
  // the larger of the 16-byte and per-element geometries: the call may take either
  // (the pointers' alignment is not known here)
  RowGeom g;
  if (M <= 0 || N <= 0 || ld < N || !bwd_geom(dtype, N, ld, true, &g)) return 0;
  int groups = bwd_groups(M, g);
  RowGeom gs;
  if (bwd_geom(dtype, N, ld, false, &gs) && bwd_groups(M, gs) > groups) groups = bwd_groups(M, gs);
  return (size_t)groups * 2 * N * sizeof(float);
}

int icpp_layernorm_bwd(int dtype, const void* DY, const void* X, const void* W, const float* mean, const float* rstd,
                       void* DX, void* DW, void* DB, int M, int N, int ld, void* workspace, size_t ws_bytes,
                       void* stream) {
  if (!DY || !X || !W || !mean || !rstd || !DX || !DW || !DB) return set_error(ICPP_E_ARG, "icpp_layernorm_bwd: null tensor");
  if (int rc = check_rows("icpp_layernorm_bwd: bad dtype or shape", dtype, M, N, ld, ld)) return rc;
  RowGeom g;
  const bool al = aligned16(DY) && aligned16(X) && aligned16(W) && aligned16(DX);
  if (!bwd_geom(dtype, N, ld, al, &g)) return set_error(ICPP_E_SHAPE, "icpp_layernorm_bwd: N too large");
  const size_t need = (size_t)bwd_groups(M, g) * 2 * N * sizeof(float);
  if (!workspace || ws_bytes < need || !aligned16(workspace))
    return set_error(ICPP_E_WORKSPACE, "icpp_layernorm_bwd: workspace too small (see icpp_layernorm_bwd_workspace_bytes)");
  hipStream_t s = (hipStream_t)stream;
  float* part = (float*)workspace;
  if (dtype == ICPP_F16) return ln_bwd_t<_Float16>(DY, X, W, mean, rstd, DX, DW, DB, M, N, ld, g, part, s);
  if (dtype == ICPP_BF16) return ln_bwd_t<__bf16>(DY, X, W, mean, rstd, DX, DW, DB, M, N, ld, g, part, s);
  return ln_bwd_t<float>(DY, X, W, mean, rstd, DX, DW, DB, M, N, ld, g, part, s);
}

int icpp_softmax(int dtype, const void* X, void* Y, int M, int N, int ldx, int ldy, void* stream) {
  if (!X || !Y) return set_error(ICPP_E_ARG, "icpp_softmax: null tensor");
  if (int rc = check_rows("icpp_softmax: bad dtype or shape", dtype, M, N, ldx, ldy)) return rc;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ICPP_F16) return softmax_t<_Float16>(X, Y, M, N, ldx, ldy, s);
  if (dtype == ICPP_BF16) return softmax_t<__bf16>(X, Y, M, N, ldx, ldy, s);
  return softmax_t<float>(X, Y, M, N, ldx, ldy, s);
}

int icpp_softmax_scaled_masked(int dtype, const void* X, void* Y, const void* mask, float scale, int M, int N, int ldx,
                               int ldy, int mask_rows, void* stream) {
  if (!X || !Y) return set_error(ICPP_E_ARG, "icpp_softmax_scaled_masked: null tensor");
  if (int rc = check_rows("icpp_softmax_scaled_masked: bad dtype or shape", dtype, M, N, ldx, ldy)) return rc;
  if (mask != nullptr && mask_rows <= 0) return set_error(ICPP_E_SHAPE, "icpp_softmax_scaled_masked: mask_rows must be > 0");
  if (!(scale == scale) || scale == INFINITY || scale == -INFINITY)
    return set_error(ICPP_E_ARG, "icpp_softmax_scaled_masked: scale must be finite");
  hipStream_t s = (hipStream_t)stream;
  const int mr = mask != nullptr ? mask_rows : 1;
  if (dtype == ICPP_F16) return softmax_t<_Float16>(X, Y, M, N, ldx, ldy, s, true, mask, scale, mr);
  if (dtype == ICPP_BF16) return softmax_t<__bf16>(X, Y, M, N, ldx, ldy, s, true, mask, scale, mr);
  return softmax_t<float>(X, Y, M, N, ldx, ldy, s, true, mask, scale, mr);
}

// Attention head layout (head_dim 64): see qkv_split_heads_kernel / merge_heads_kernel.
int icpp_qkv_split_heads(int dtype, const void* QKV, const void* bias, void* Q, void* K, void* V, int batch,
                         int seq, int heads, int head_dim, int layout, void* stream) {
  if (!QKV || !Q || !K || !V) return set_error(ICPP_E_ARG, "icpp_qkv_split_heads: null tensor");
  if (layout != 0 && layout != 1) return set_error(ICPP_E_ARG, "icpp_qkv_split_heads: layout must be 0 or 1");
  if (dtype != ICPP_F16 && dtype != ICPP_BF16) return set_error(ICPP_E_ARG, "icpp_qkv_split_heads: dtype must be f16 or bf16");
  if (head_dim != HD) return set_error(ICPP_E_SHAPE, "icpp_qkv_split_heads: head_dim must be 64");
  if (batch <= 0 || seq <= 0 || heads <= 0 || (long long)batch * seq * heads * 3 * HD > 0x7FFFFFFFll)
    return set_error(ICPP_E_SHAPE, "icpp_qkv_split_heads: bad or too large shape");
  if (!aligned16(QKV) || (bias && !aligned16(bias)) || !aligned16(Q) || !aligned16(K) || !aligned16(V))
    return set_error(ICPP_E_ARG, "icpp_qkv_split_heads: pointers must be 16-byte aligned");
  const dim3 grid((seq + HD - 1) / HD, heads, batch);
  if (batch > 65535 || heads > 65535) return set_error(ICPP_E_SHAPE, "icpp_qkv_split_heads: grid too large");
  hipStream_t s = (hipStream_t)stream;
  auto launch = [&](auto tag, auto TPc) {
    typedef decltype(tag) T;
    hipLaunchKernelGGL((qkv_split_heads_kernel<T, decltype(TPc)::value>), grid, dim3(256), 0, s, (const T*)QKV,
                       (const T*)bias, (T*)Q, (T*)K, (T*)V, seq, heads);
  };
  if (dtype == ICPP_F16) {
    if (layout == 0) launch(_Float16{}, std::integral_constant<int, 1>{});
    else launch(_Float16{}, std::integral_constant<int, 2>{});
  } else {
    if (layout == 0) launch(__bf16{}, std::integral_constant<int, 1>{});
    else launch(__bf16{}, std::integral_constant<int, 2>{});
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ICPP_OK : set_error((int)e, hipGetErrorString(e));
}

int icpp_merge_heads(int dtype, const void* X, void* Y, int batch, int seq, int heads, int head_dim, void* stream) {
  if (!X || !Y) return set_error(ICPP_E_ARG, "icpp_merge_heads: null tensor");
  if (dtype != ICPP_F16 && dtype != ICPP_BF16) return set_error(ICPP_E_ARG, "icpp_merge_heads: dtype must be f16 or bf16");
  if (head_dim != HD) return set_error(ICPP_E_SHAPE, "icpp_merge_heads: head_dim must be 64");
  if (batch <= 0 || seq <= 0 || heads <= 0 || (long long)batch * seq * heads * HD > 0x7FFFFFFFll)
    return set_error(ICPP_E_SHAPE, "icpp_merge_heads: bad or too large shape");
  if (!aligned16(X) || !aligned16(Y)) return set_error(ICPP_E_ARG, "icpp_merge_heads: pointers must be 16-byte aligned");
  const long long chunks = (long long)batch * seq * heads * (HD / 8);
  const int blocks = (int)std::min<long long>((chunks + 255) / 256, 4096);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ICPP_F16)
    hipLaunchKernelGGL(merge_heads_kernel<_Float16>, dim3(blocks), dim3(256), 0, s, (const _Float16*)X, (_Float16*)Y,
                       batch, seq, heads);
  else
    hipLaunchKernelGGL(merge_heads_kernel<__bf16>, dim3(blocks), dim3(256), 0, s, (const __bf16*)X, (__bf16*)Y,
                       batch, seq, heads);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ICPP_OK : set_error((int)e, hipGetErrorString(e));
}

}  // extern "C"
