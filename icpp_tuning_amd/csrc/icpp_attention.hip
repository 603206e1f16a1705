// Fused attention forward of the BERT layer, head_dim 64:
//   O[b, s, h*64] = softmax(Q K^T * scale + mask) V   per (batch, head)
// (evaluation/end2end.py:59-73: baddbmm(q, k) * 1/sqrt(d), + causal mask, softmax,
// einsum with v, reshaped to [b, t, h*d]), one launch instead of two batched
// products, a softmax pass and the context merge.
//
// A wave owns 16 queries of one (batch, head).  Up to 128 keys the four waves of
// a workgroup never synchronise; longer sequences use a variant that shares K and
// V^T through LDS and passes P through LDS one 32-key tile at a time (below).
// Per wave:
//   1. S = Q K^T for all keys with 16x16x32 MFMAs: the 16 x 64 query block stays
//      in two fragments, every 16-key tile of K [seq, 64] is read straight from
//      global memory (16 contiguous bytes per lane).  S stays in registers (this
//      direct kernel serves up to 128 keys), scaled and masked in fp32.
//   2. Row softmax over the registers: each query row is spread over the 4 lanes
//      r, r+16, r+32, r+48, so the max and the sum take two cross-lane steps.
//   3. P is rounded to the data type and written to the wave's LDS rows (stride
//      seq + 8 elements, so the 16 rows of a fragment read land in distinct banks),
//      then read back as A fragments for O = P V with V^T [64, seq] as the B
//      operand (16 contiguous bytes per lane again).
//   4. O goes out in the merged [batch*seq, heads*64] layout, 8 bytes per lane.
// Limits: seq a multiple of 32, at most 512; the mask, if any, is [seq, seq] in
// the data type (added to every (batch, head)).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "icpp_kernels.hpp"
#include "../../include/icpp_hip.h"

namespace icpp {
int set_last_error(int code, const char* msg);  // icpp_abi.hip: the library's last-error buffer

namespace {

constexpr int AD = 64;        // head_dim
constexpr int ATT_MAX_SEQ = 512;

template <int DT, int NT_MAX, bool HAS_MASK>
__global__ void __launch_bounds__(256)
attention_fwd_kernel(const void* Qp, const void* Kp, const void* VTp, const void* Mp, void* Op, int seq, int heads,
                     float scale) {
  typedef typename DTraits<DT>::T T;
  typedef Mfma<DT, 16> MF;
  typedef T t4 __attribute__((ext_vector_type(4)));
  constexpr int PST_MAX = NT_MAX * 16 + 8;  // LDS row stride bound (elements)
  __shared__ __attribute__((aligned(16))) T plds[4][16 * PST_MAX];
  const T* Q = (const T*)Qp;
  const T* K = (const T*)Kp;
  const T* VT = (const T*)VTp;
  const T* M = (const T*)Mp;
  T* O = (T*)Op;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int bh = blockIdx.y;
  const int bb = bh / heads, hh = bh - bb * heads;
  const int q0 = blockIdx.x * 64 + wave * 16;
  if (q0 >= seq) return;  // no workgroup barrier below: an idle wave simply leaves
  const int NT = seq / 16;
  const int PST = seq + 8;
  const int q = q0 + r;  // this lane's query (A-operand row and output row)
  const bool qok = q < seq;

  i32x4 qf[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
    qf[ks] = qok ? *reinterpret_cast<const i32x4*>(Q + ((size_t)bh * seq + q) * AD + ks * 32 + g * 8)
                 : i32x4{0, 0, 0, 0};

  // 1. scores: lane holds S[q][kt*16 + 4g + j].  Every load is unconditional -- tiles
  // past the last one re-read the last tile and rows past seq read row seq-1, results
  // discarded -- so the unrolled loop has no branches and all K and mask loads can be
  // in flight together instead of one round trip per tile.
  const int qc = qok ? q : seq - 1;
  float sv[NT_MAX][4];
  constexpr int KB = 8;  // key tiles whose loads are all issued before their MFMAs
#pragma unroll
  for (int kb = 0; kb < NT_MAX; kb += KB) {
    i32x4 kf[KB][2];
    t4 m4[KB];
#pragma unroll
    for (int t = 0; t < KB; ++t) {
      const int kt = kb + t;
      const int ktc = kt < NT ? kt : NT - 1;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        kf[t][ks] = *reinterpret_cast<const i32x4*>(K + ((size_t)bh * seq + ktc * 16 + r) * AD + ks * 32 + g * 8);
      if constexpr (HAS_MASK) m4[t] = *reinterpret_cast<const t4*>(M + (size_t)qc * seq + ktc * 16 + 4 * g);
    }
#pragma unroll
    for (int t = 0; t < KB; ++t) {
      const int kt = kb + t;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) acc = MF::run(kf[t][ks], qf[ks], acc);
      f32x4 mk = {0.f, 0.f, 0.f, 0.f};
      if constexpr (HAS_MASK) mk = f32x4{(float)m4[t][0], (float)m4[t][1], (float)m4[t][2], (float)m4[t][3]};
#pragma unroll
      for (int j = 0; j < 4; ++j) sv[kt][j] = kt < NT ? fmaf(acc[j], scale, mk[j]) : -INFINITY;
    }
  }

  // 2. row softmax (fp32): the row's other values sit in lanes r ^ 16, r ^ 32
  float mx = -INFINITY;
#pragma unroll
  for (int kt = 0; kt < NT_MAX; ++kt)
#pragma unroll
    for (int j = 0; j < 4; ++j) mx = fmaxf(mx, sv[kt][j]);
  mx = fmaxf(mx, __shfl_xor(mx, 16));
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  float sum = 0.f;
#pragma unroll
  for (int kt = 0; kt < NT_MAX; ++kt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float e = kt < NT ? __expf(sv[kt][j] - mx) : 0.f;
      sv[kt][j] = e;
      sum += e;
    }
  sum += __shfl_xor(sum, 16);
  sum += __shfl_xor(sum, 32);
  const float inv = 1.f / sum;

  // 3. P -> this wave's LDS rows, then O = P V
  T* prow = plds[wave];
#pragma unroll
  for (int kt = 0; kt < NT_MAX; ++kt)
    if (kt < NT) {
      const t4 pv = {(T)(sv[kt][0] * inv), (T)(sv[kt][1] * inv), (T)(sv[kt][2] * inv), (T)(sv[kt][3] * inv)};
      *reinterpret_cast<t4*>(prow + r * PST + kt * 16 + 4 * g) = pv;
    }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  f32x4 oacc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) oacc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  // past the last 32-key step the V^T read is clamped and P is zero, so the MFMA adds nothing
#pragma unroll
  for (int kk = 0; kk < NT_MAX / 2; ++kk) {
    const bool live = 2 * kk < NT;
    const int kkc = live ? kk : NT / 2 - 1;
    const i32x4 p_raw = *reinterpret_cast<const i32x4*>(prow + r * PST + kkc * 32 + g * 8);
    const i32x4 pf = live ? p_raw : i32x4{0, 0, 0, 0};
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const i32x4 vf =
          *reinterpret_cast<const i32x4*>(VT + ((size_t)bh * AD + dt * 16 + r) * seq + kkc * 32 + g * 8);
      oacc[dt] = MF::run(vf, pf, oacc[dt]);
    }
  }

  // 4. O[bb*seq + q][hh*64 + dt*16 + 4g + j]
  if (qok) {
    T* orow = O + ((size_t)bb * seq + q) * ((size_t)heads * AD) + hh * AD;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const t4 ov = {(T)oacc[dt][0], (T)oacc[dt][1], (T)oacc[dt][2], (T)oacc[dt][3]};
      *reinterpret_cast<t4*>(orow + dt * 16 + 4 * g) = ov;
    }
  }
}

// Long sequences (up to 512 keys): the same per-wave work, but the four waves share
// K and V^T through LDS in chunks of 128 keys (each loaded once per workgroup instead
// of once per wave), with two workgroup barriers per chunk.  Every wave takes part in
// the loads and barriers; a wave past the last query only skips the arithmetic.
constexpr int CH = 128;          // keys per chunk
constexpr int KST = AD + 8;      // K chunk row stride (elements): 16 key rows of a fragment read hit distinct banks
constexpr int VST = CH + 8;      // V^T chunk row stride (elements)
template <int DT>
__global__ void __launch_bounds__(256)
attention_fwd_staged_kernel(const void* Qp, const void* Kp, const void* VTp, const void* Mp, void* Op, int seq,
                            int heads, float scale) {
  typedef typename DTraits<DT>::T T;
  typedef Mfma<DT, 16> MF;
  typedef T t4 __attribute__((ext_vector_type(4)));
  constexpr int NT_MAX = ATT_MAX_SEQ / 16, NC = ATT_MAX_SEQ / CH, PTS = 40;
  // P goes through LDS 32 keys at a time (a 16 x 32 tile per wave), so the workgroup's
  // LDS is ~23 KB and occupancy is set by registers rather than by whole P rows
  __shared__ __attribute__((aligned(16))) T plds[4][16 * PTS];
  __shared__ __attribute__((aligned(16))) T kv[CH * KST > AD * VST ? CH * KST : AD * VST];
  const T* Q = (const T*)Qp;
  const T* K = (const T*)Kp;
  const T* VT = (const T*)VTp;
  const T* M = (const T*)Mp;
  T* O = (T*)Op;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int bh = blockIdx.y;
  const int bb = bh / heads, hh = bh - bb * heads;
  const int q0 = blockIdx.x * 64 + wave * 16;
  const bool active = q0 < seq;
  const int NT = seq / 16;
  const int q = q0 + r;
  const bool qok = q < seq;

  i32x4 qf[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
    qf[ks] = qok ? *reinterpret_cast<const i32x4*>(Q + ((size_t)bh * seq + q) * AD + ks * 32 + g * 8)
                 : i32x4{0, 0, 0, 0};

  float sv[NT_MAX][4];
#pragma unroll
  for (int kt = 0; kt < NT_MAX; ++kt)
#pragma unroll
    for (int j = 0; j < 4; ++j) sv[kt][j] = -INFINITY;
  // 1. scores, one 128-key chunk of K at a time: 128 rows x 8 chunks of 16 bytes, 4 per thread
  // chunk c+1 is loaded into registers while chunk c multiplies
  i32x4 pre[4];
  auto load_k = [&](int c) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int x = tid + 256 * i, key = c * CH + (x >> 3);
      if (key < seq) pre[i] = *reinterpret_cast<const i32x4*>(K + ((size_t)bh * seq + key) * AD + (x & 7) * 8);
    }
  };
  auto load_v = [&](int c) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int x = tid + 256 * i, key = c * CH + (x & 15) * 8;
      if (key < seq) pre[i] = *reinterpret_cast<const i32x4*>(VT + ((size_t)bh * AD + (x >> 4)) * seq + key);
    }
  };
  load_k(0);
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    if (c * CH < seq) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int x = tid + 256 * i;
        if (c * CH + (x >> 3) < seq) *reinterpret_cast<i32x4*>(kv + (x >> 3) * KST + (x & 7) * 8) = pre[i];
      }
      __syncthreads();
      if ((c + 1) * CH < seq) load_k(c + 1);
      else load_v(0);
      if (active) {
#pragma unroll
        for (int t = 0; t < CH / 16; ++t) {
          const int kt = c * (CH / 16) + t;
          if (kt < NT) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
              const i32x4 kf = *reinterpret_cast<const i32x4*>(kv + (t * 16 + r) * KST + ks * 32 + g * 8);
              acc = MF::run(kf, qf[ks], acc);
            }
            f32x4 mk = {0.f, 0.f, 0.f, 0.f};
            if (M != nullptr && qok) {
              const t4 m4 = *reinterpret_cast<const t4*>(M + (size_t)q * seq + kt * 16 + 4 * g);
              mk = f32x4{(float)m4[0], (float)m4[1], (float)m4[2], (float)m4[3]};
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) sv[kt][j] = fmaf(acc[j], scale, mk[j]);
          }
        }
      }
      __syncthreads();
    }
  }

  // 2. row softmax
  float mx = -INFINITY;
#pragma unroll
  for (int kt = 0; kt < NT_MAX; ++kt)
#pragma unroll
    for (int j = 0; j < 4; ++j) mx = fmaxf(mx, sv[kt][j]);
  mx = fmaxf(mx, __shfl_xor(mx, 16));
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  float sum = 0.f;
#pragma unroll
  for (int kt = 0; kt < NT_MAX; ++kt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float e = kt < NT ? __expf(sv[kt][j] - mx) : 0.f;
      sv[kt][j] = e;
      sum += e;
    }
  sum += __shfl_xor(sum, 16);
  sum += __shfl_xor(sum, 32);
  const float inv = 1.f / sum;
  T* ptile = plds[wave];

  // 3. O = P V, one 128-key chunk of V^T at a time: 64 rows x 16 chunks of 16 bytes, 4 per thread
  f32x4 oacc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) oacc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    if (c * CH < seq) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int x = tid + 256 * i;
        if (c * CH + (x & 15) * 8 < seq) *reinterpret_cast<i32x4*>(kv + (x >> 4) * VST + (x & 15) * 8) = pre[i];
      }
      __syncthreads();
      if ((c + 1) * CH < seq) load_v(c + 1);
      if (active) {
#pragma unroll
        for (int u = 0; u < CH / 32; ++u) {
          const int kk = c * (CH / 32) + u;
          if (2 * kk < NT) {  // seq % 32 == 0, so tile 2kk+1 is live too
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const float* e = sv[2 * kk + h];
              const t4 pv = {(T)(e[0] * inv), (T)(e[1] * inv), (T)(e[2] * inv), (T)(e[3] * inv)};
              *reinterpret_cast<t4*>(ptile + r * PTS + h * 16 + 4 * g) = pv;
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            const i32x4 pf = *reinterpret_cast<const i32x4*>(ptile + r * PTS + g * 8);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
              const i32x4 vf = *reinterpret_cast<const i32x4*>(kv + (dt * 16 + r) * VST + u * 32 + g * 8);
              oacc[dt] = MF::run(vf, pf, oacc[dt]);
            }
          }
        }
      }
      __syncthreads();
    }
  }

  if (qok) {
    T* orow = O + ((size_t)bb * seq + q) * ((size_t)heads * AD) + hh * AD;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const t4 ov = {(T)oacc[dt][0], (T)oacc[dt][1], (T)oacc[dt][2], (T)oacc[dt][3]};
      *reinterpret_cast<t4*>(orow + dt * 16 + 4 * g) = ov;
    }
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <int DT>
hipError_t launch_attention(const void* Q, const void* K, const void* VT, const void* M, void* O, int batch, int seq,
                            int heads, float scale, hipStream_t s) {
  const dim3 grid((seq + 63) / 64, batch * heads);
  auto direct = [&](auto NTc, auto MASKc) {
    hipLaunchKernelGGL((attention_fwd_kernel<DT, decltype(NTc)::value, decltype(MASKc)::value>), grid, dim3(256), 0, s,
                       Q, K, VT, M, O, seq, heads, scale);
  };
  if (seq <= 128) {
    if (M) direct(std::integral_constant<int, 8>{}, std::true_type{});
    else direct(std::integral_constant<int, 8>{}, std::false_type{});
  } else  // from 160 keys the shared-K/V staged kernel is the faster one (2.6 us less at 256)
    hipLaunchKernelGGL((attention_fwd_staged_kernel<DT>), grid, dim3(256), 0, s, Q, K, VT, M, O, seq, heads, scale);
  return hipGetLastError();
}

}  // namespace
}  // namespace icpp

using namespace icpp;

extern "C" {

int icpp_attention_fwd(int dtype, const void* Q, const void* K, const void* VT, const void* mask, float scale, void* O,
                       int batch, int seq, int heads, int head_dim, void* stream) {
  if (!Q || !K || !VT || !O) return set_last_error(ICPP_E_ARG, "icpp_attention_fwd: null tensor");
  if (dtype != ICPP_F16 && dtype != ICPP_BF16) return set_last_error(ICPP_E_ARG, "icpp_attention_fwd: dtype must be f16 or bf16");
  if (head_dim != AD) return set_last_error(ICPP_E_SHAPE, "icpp_attention_fwd: head_dim must be 64");
  if (batch <= 0 || heads <= 0 || seq <= 0 || seq % 32 || seq > ATT_MAX_SEQ || batch * (long long)heads > 65535 ||
      (long long)batch * heads * seq * AD > 0x7FFFFFFFll)
    return set_last_error(ICPP_E_SHAPE, "icpp_attention_fwd: need seq a multiple of 32 up to 512 and batch*heads <= 65535");
  if (!(scale == scale) || scale == INFINITY || scale == -INFINITY)
    return set_last_error(ICPP_E_ARG, "icpp_attention_fwd: scale must be finite");
  if (!aligned16(Q) || !aligned16(K) || !aligned16(VT) || !aligned16(O) || (mask && !aligned16(mask)))
    return set_last_error(ICPP_E_ARG, "icpp_attention_fwd: pointers must be 16-byte aligned");
  const hipError_t e = dtype == ICPP_F16
                           ? launch_attention<DT_F16>(Q, K, VT, mask, O, batch, seq, heads, scale, (hipStream_t)stream)
                           : launch_attention<DT_BF16>(Q, K, VT, mask, O, batch, seq, heads, scale, (hipStream_t)stream);
  return e == hipSuccess ? ICPP_OK : set_last_error((int)e, hipGetErrorString(e));
}

}  // extern "C"
