// fp8 e4m3 GEMM + bias + activation for decode-sized M (1..32) over pre-packed weights.
//
// The split-K kernels read B [K, N] (N contiguous) in tiles: at M <= 32 a launch
// needs K split across workgroups to keep enough CUs streaming B, and the split
// costs a second launch that sums the fp32 partials.  With the weights packed once
// (static weights in serving) so that every 16-column block is one contiguous run
// over K, a workgroup streams its column block sequentially, its four waves take
// interleaved 128-deep K steps, and the partial sums meet in LDS: one launch, no
// partials in memory.
//
// Packed layout (icpp_fp8_pack_b): for column block nb (columns 16 nb .. +15) and
// K step s (rows 128 s .. +127), 2 KiB at byte ((nb * S + s) * 64 + l) * 32, where
// lane l's 32 bytes are B[128 s + 32 (l / 16) + t][16 nb + l % 16], t = 0..31 --
// exactly the operand lane l of a 16x16x128 fp8 MFMA holds (row l % 16, K slice
// (l / 16) * 32 .. +32), so each lane reads its fragment with two 16-byte loads
// and a wave reads 2 KiB of consecutive bytes.  S = K / 128.
//
// The MFMA takes the B block as its first operand (rows = output columns n) and
// A as its second (columns = output rows m): result lane l holds m = l % 16 and
// n = 16 nb + 4 (l / 16) + 0..3, four consecutive outputs of one row per lane.
// M = 17..32 runs two row tiles per wave (rows 16 j + l % 16), both against the
// same B fragment.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "icpp_hip.h"
#include "icpp_kernels.hpp"

namespace icpp {
int set_last_error(int code, const char* msg);  // icpp_abi.hip
}

namespace {

using namespace icpp;

constexpr int kDecodeWaves = 4;   // waves per workgroup, splitting the K steps
constexpr int kDecodeUnroll = 8;  // K steps per wave whose loads are in flight together

// MT row tiles of 16 (M <= 16 MT): each K step's B fragment meets MT A fragments.
template <int ACT, int MT>
__global__ void __launch_bounds__(64 * kDecodeWaves) __attribute__((amdgpu_waves_per_eu(1, 2)))
fp8_decode_kernel(const uint8_t* __restrict__ A, const uint8_t* __restrict__ Bp, const float* __restrict__ bias,
                  __bf16* __restrict__ C, int M, int N, int K, float alpha) {
  typedef Mfma<DT_FP8, 16> Op;
  constexpr int U = kDecodeUnroll;  // steps per group, their fragments all in registers  // steps per group: fragments in registers
  const int nb = blockIdx.x;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int S = K >> 7;
  // rows m >= M lie past the descriptor's range: their loads return zeros
  const __amdgpu_buffer_rsrc_t ar = make_rsrc(A, (uint32_t)(M * K));
  const __amdgpu_buffer_rsrc_t br = make_rsrc(Bp + (size_t)nb * S * 2048, (uint32_t)(S * 2048));
  const uint32_t a_lane = (uint32_t)((lane & 15) * K + (lane >> 4) * 32);
  const uint32_t b_lane = (uint32_t)(lane * 32);
  f32x4 acc[MT];
#pragma unroll
  for (int j = 0; j < MT; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // Groups of U steps, every load of a group issued before its MFMAs.  Steps past the
  // end (the last group of a wave) read from an offset past both descriptors' ranges,
  // so their fragments are zeros and add nothing.
  for (int s = wave; s < S; s += U * kDecodeWaves) {
    Op::Frag af[U][MT], bf[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int su = s + u * kDecodeWaves;
      const uint32_t bo = su < S ? b_lane + (uint32_t)su * 2048 : ICPP_OOB_OFFSET;
      const i32x4 b0 = buf_load16(br, bo), b1 = buf_load16(br, bo + 16);
      bf[u] = Op::Frag{b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
#pragma unroll
      for (int j = 0; j < MT; ++j) {
        const uint32_t ao = su < S ? a_lane + (uint32_t)(16 * j * K) + (uint32_t)su * 128 : ICPP_OOB_OFFSET;
        const i32x4 a0 = buf_load16(ar, ao), a1 = buf_load16(ar, ao + 16);
        af[u][j] = Op::Frag{a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
      }
    }
    // keep the group's loads ahead of its MFMAs (the scheduler would otherwise trickle
    // them in between, one K step in flight at a time)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < MT; ++j) acc[j] = Op::run(bf[u], af[u][j], acc[j]);
  }
  // the waves' partial sums meet in LDS, added in wave order
  __shared__ f32x4 part[kDecodeWaves][MT][64];
#pragma unroll
  for (int j = 0; j < MT; ++j) part[wave][j][lane] = acc[j];
  __syncthreads();
  if (wave != 0) return;
  const int n = nb * 16 + 4 * (lane >> 4);
  const f32x4 bv = bias ? *reinterpret_cast<const f32x4*>(bias + n) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < MT; ++j) {
    f32x4 v = part[0][j][lane];
#pragma unroll
    for (int w = 1; w < kDecodeWaves; ++w) v += part[w][j][lane];
    const int m = 16 * j + (lane & 15);
    if (m >= M) continue;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = act_fn<ACT>(v[e] * alpha + bv[e]);
    Vec4Store<__bf16>::st(C + (size_t)m * N + n, v);
  }
}

// One thread per 16 bytes of the packed layout: a strided gather from B [K, N].
__global__ void __launch_bounds__(256)
fp8_pack_b_kernel(const uint8_t* __restrict__ B, uint8_t* __restrict__ Bp, int K, int N) {
  const size_t chunks = (size_t)K * N / 16;
  const int S = K >> 7;
  for (size_t c = (size_t)blockIdx.x * blockDim.x + threadIdx.x; c < chunks; c += (size_t)gridDim.x * blockDim.x) {
    const size_t q = c * 16;
    const int t0 = (int)(q & 31);
    const int l = (int)((q >> 5) & 63);
    const size_t blk = q >> 11;  // nb * S + s
    const int s = (int)(blk % S);
    const int nb = (int)(blk / S);
    const size_t k0 = (size_t)s * 128 + (l >> 4) * 32 + t0;
    const size_t col = (size_t)nb * 16 + (l & 15);
    uint8_t v[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) v[t] = B[(k0 + t) * N + col];
    i32x4 w;
    __builtin_memcpy(&w, v, 16);
    *reinterpret_cast<i32x4*>(Bp + q) = w;
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

extern "C" {

int icpp_fp8_pack_b(const void* B, void* Bp, int K, int N, void* stream) {
  if (!B || !Bp) return icpp::set_last_error(ICPP_E_ARG, "icpp_fp8_pack_b: null tensor");
  if (K <= 0 || N <= 0 || K % 128 || N % 16)
    return icpp::set_last_error(ICPP_E_SHAPE, "icpp_fp8_pack_b: need K > 0, K % 128 == 0, N > 0 and N % 16 == 0");
  if (!aligned16(Bp)) return icpp::set_last_error(ICPP_E_ARG, "icpp_fp8_pack_b: Bp must be 16-byte aligned");
  const size_t chunks = (size_t)K * N / 16;
  const int blocks = (int)std::min<size_t>((chunks + 255) / 256, 8192);
  hipLaunchKernelGGL(fp8_pack_b_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (const uint8_t*)B,
                     (uint8_t*)Bp, K, N);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ICPP_OK : icpp::set_last_error((int)e, "icpp_fp8_pack_b: launch failed");
}

int icpp_fp8_gemm_packed(const void* A, const void* Bp, const void* bias, void* C, int M, int N, int K, int act,
                         float scale_a, float scale_b, void* stream) {
  if (!A || !Bp || !C) return icpp::set_last_error(ICPP_E_ARG, "icpp_fp8_gemm_packed: null tensor");
  if (M < 1 || M > 32) return icpp::set_last_error(ICPP_E_SHAPE, "icpp_fp8_gemm_packed: M must be 1..32");
  if (K <= 0 || N <= 0 || K % 128 || N % 16)
    return icpp::set_last_error(ICPP_E_SHAPE, "icpp_fp8_gemm_packed: need K > 0, K % 128 == 0, N > 0 and N % 16 == 0");
  if ((size_t)M * K >= ((size_t)1 << 31) || (size_t)K * 32 >= ((size_t)1 << 31))
    return icpp::set_last_error(ICPP_E_SHAPE, "icpp_fp8_gemm_packed: K too large");
  if (act < ICPP_ACT_NONE || act > ICPP_ACT_GELU_ERF)
    return icpp::set_last_error(ICPP_E_ARG, "icpp_fp8_gemm_packed: unknown activation");
  if (!aligned16(A) || !aligned16(Bp) || !aligned16(C) || (bias && !aligned16(bias)))
    return icpp::set_last_error(ICPP_E_ARG, "icpp_fp8_gemm_packed: pointers must be 16-byte aligned");
  const float alpha = scale_a * scale_b;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid(N / 16), block(64 * kDecodeWaves);
  const uint8_t* a = (const uint8_t*)A;
  const uint8_t* b = (const uint8_t*)Bp;
  const float* bi = (const float*)bias;
  __bf16* c = (__bf16*)C;
  auto launch = [&](auto MT) {
    constexpr int mt = decltype(MT)::value;
    switch (act) {
      case ICPP_ACT_RELU: hipLaunchKernelGGL((fp8_decode_kernel<ACT_RELU, mt>), grid, block, 0, s, a, b, bi, c, M, N, K, alpha); break;
      case ICPP_ACT_GELU_TANH: hipLaunchKernelGGL((fp8_decode_kernel<ACT_GELU_TANH, mt>), grid, block, 0, s, a, b, bi, c, M, N, K, alpha); break;
      case ICPP_ACT_SILU: hipLaunchKernelGGL((fp8_decode_kernel<ACT_SILU, mt>), grid, block, 0, s, a, b, bi, c, M, N, K, alpha); break;
      case ICPP_ACT_GELU_ERF: hipLaunchKernelGGL((fp8_decode_kernel<ACT_GELU_ERF, mt>), grid, block, 0, s, a, b, bi, c, M, N, K, alpha); break;
      default: hipLaunchKernelGGL((fp8_decode_kernel<ACT_NONE, mt>), grid, block, 0, s, a, b, bi, c, M, N, K, alpha); break;
    }
  };
  if (M <= 16) launch(std::integral_constant<int, 1>{});
  else launch(std::integral_constant<int, 2>{});
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ICPP_OK : icpp::set_last_error((int)e, "icpp_fp8_gemm_packed: launch failed");
}

}  // extern "C"
