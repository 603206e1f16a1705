// Instance registry shared by the generated instance translation units and the
// C ABI.  Each AOT-compiled tile configuration registers one Instance from a
// static initializer when the shared library is loaded.
#pragma once
#include "icpp_kernels.hpp"
#include "../../include/icpp_hip.h"

namespace icpp {

typedef hipError_t (*LaunchFn)(const KArgs&, dim3, hipStream_t);

struct Instance {
  icpp_tile_t tile;
  int epi;
  int aload;
  int wave_tile_n;
  LaunchFn launch;         // conv instances: the per-tile-tap gather (C % block_k == 0)
  LaunchFn launch_gather;  // conv instances: the per-chunk gather (any C % 8 == 0); else null
  LaunchFn launch_halo;    // conv instances: the input-halo loader (3x3 stride 1 pad 1, C == block_k); or null
  int halo_bytes;          // its halo capacity (halo_cap(block_m))
  // f16 dense GEMM instances: the same tile with the co-resident LayerNorm epilogue
  // (EPI_LN_CR), its workgroups resident per CU, and the LDS bytes of one stage array
  // (the row block's statistics are gathered into it); else null / 0
  LaunchFn launch_ln_cr;
  int (*resident_ln_cr)();
  int ln_cr_stage_bytes;
};

int register_instance(const Instance& inst);

template <int DT, int BM, int BN, int BK, int WM, int WN, int MF, int ST, int EPI, int AL>
hipError_t launch_instance(const KArgs& a, dim3 grid, hipStream_t s) {
  hipLaunchKernelGGL((gemm_kernel<DT, BM, BN, BK, WM, WN, MF, ST, EPI, AL>), grid, dim3(WM * WN * 64), 0, s, a);
  return hipGetLastError();
}

// Workgroups of the kernel one CU holds at once (registers, LDS, waves), 0 if unknown.
template <int DT, int BM, int BN, int BK, int WM, int WN, int MF, int ST, int EPI, int AL>
int resident_per_cu() {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &n, reinterpret_cast<const void*>(&gemm_kernel<DT, BM, BN, BK, WM, WN, MF, ST, EPI, AL>), WM * WN * 64, 0) !=
      hipSuccess)
    return 0;
  return n;
}

template <int DT, int BM, int BN, int BK, int WM, int WN, int MF, int ST, int EPI, int AL>
Instance make_instance(int family, const char* name) {
  typedef Tile<DT, BM, BN, BK, WM, WN, MF, ST> G;
  Instance in{};
  in.tile.family = family;
  in.tile.dtype = DT;
  in.tile.block_m = BM;
  in.tile.block_n = BN;
  in.tile.block_k = BK;
  in.tile.waves_m = WM;
  in.tile.waves_n = WN;
  in.tile.stages = ST;
  in.tile.mfma_m = MF;
  in.tile.mfma_n = MF;
  in.tile.mfma_k = Mfma<DT, MF>::KI;
  in.tile.lds_bytes = G::LDS_BYTES;
  in.tile.threads = G::THREADS;
  int i = 0;
  for (; name[i] && i < (int)sizeof(in.tile.name) - 1; ++i) in.tile.name[i] = name[i];
  in.tile.name[i] = 0;
  in.epi = EPI;
  in.aload = AL;
  in.wave_tile_n = G::WTN;
  if constexpr ((AL & 7) == A_IM2COL) {
    constexpr int PPB = AL & A_PP;  // the schedule bit carries over to every conv loader
    in.launch = &launch_instance<DT, BM, BN, BK, WM, WN, MF, ST, EPI, A_IM2COL_TAP | PPB>;
    in.launch_gather = &launch_instance<DT, BM, BN, BK, WM, WN, MF, ST, EPI, A_IM2COL | PPB>;
    constexpr bool halo_fits = G::ESZ == 2 && BK == 64 && G::B_BYTES * ST + halo_cap(BM) <= 160 * 1024;
    if constexpr (halo_fits) in.launch_halo = &launch_instance<DT, BM, BN, BK, WM, WN, MF, ST, EPI, A_HALO | PPB>;
    else in.launch_halo = nullptr;
    in.halo_bytes = halo_cap(BM);
  } else {
    in.launch = &launch_instance<DT, BM, BN, BK, WM, WN, MF, ST, EPI, AL>;
    in.launch_gather = nullptr;
  }
  if constexpr (DT == DT_F16 && EPI == EPI_STORE && (AL & 7) == A_DENSE && ST >= 2) {
    in.launch_ln_cr = &launch_instance<DT, BM, BN, BK, WM, WN, MF, ST, EPI_LN_CR, AL>;
    in.resident_ln_cr = &resident_per_cu<DT, BM, BN, BK, WM, WN, MF, ST, EPI_LN_CR, AL>;
    in.ln_cr_stage_bytes = G::STAGE_BYTES;
  } else {
    in.launch_ln_cr = nullptr;
    in.resident_ln_cr = nullptr;
    in.ln_cr_stage_bytes = 0;
  }
  return in;
}

}  // namespace icpp

#define ICPP_CAT2(a, b) a##b
#define ICPP_CAT(a, b) ICPP_CAT2(a, b)
#define ICPP_INSTANCE(FAM, DT, BM, BN, BK, WM, WN, MF, ST, EPI, AL, NAME)                                   \
  static const int ICPP_CAT(icpp_reg_, __LINE__) = icpp::register_instance(                                  \
      icpp::make_instance<DT, BM, BN, BK, WM, WN, MF, ST, EPI, AL>(FAM, NAME));
