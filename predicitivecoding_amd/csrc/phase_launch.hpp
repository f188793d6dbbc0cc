// phase_launch.hpp -- host-side entry to the phase kernels.
//
// Each (operand type, tile) instantiation of phase_kernel lives in its own
// translation unit (phase_inst.hip compiled once per combination), so the
// library's kernels build in parallel.  The host code calls them through this
// declaration; the definitions are explicit instantiations in those units.
#pragma once
#include <hip/hip_runtime.h>

#include "pc_kernels.hpp"

namespace pcd {

// Tiles with plain products that read a row-major B or a transposed A in
// place (EPI_PLAIN_KN, _MK, _MKKN): 16-bit operands on the LDS-operand tiles
// the GEMM provider uses.
constexpr bool kn_tile(int op_bytes, int bm, int bn, bool wd) {
    return op_bytes == 2 && !wd && bm == bn && (bm == 64 || bm == 128 || bm == 256);
}

// Launches phase_kernel<OP, BM, BN, epi, WD> over `grid` workgroups of
// TileCfg<BM, BN, *, WD>::NT threads on `stream` and returns the launch status.
template <typename OP, int BM, int BN, bool WD = false>
hipError_t launch_phase_tile(int epi, const ProblemSet& set, const PhaseArgs& args, int grid, hipStream_t stream);

// Launches persistent_relax_kernel<OP, BM, BN> cooperatively over `grid`
// workgroups (fp32 64 x 64 is the instantiation the library builds).
template <typename OP, int BM, int BN>
hipError_t launch_persistent_tile(const PersistArgs& args, int grid, hipStream_t stream);
extern template hipError_t launch_persistent_tile<float, 64, 64>(const PersistArgs&, int, hipStream_t);
// Workgroups of persistent_relax_kernel<float, 64, 64> one CU holds at once.
int persistent_blocks_per_cu();

#define PCD_DECLARE_TILE(OP, BM, BN)                                                                           \
    extern template hipError_t launch_phase_tile<OP, BM, BN, false>(int, const ProblemSet&, const PhaseArgs&, int, \
                                                                    hipStream_t);
#define PCD_DECLARE_OP(OP)         \
    PCD_DECLARE_TILE(OP, 32, 32)   \
    PCD_DECLARE_TILE(OP, 64, 64)   \
    PCD_DECLARE_TILE(OP, 128, 128) \
    PCD_DECLARE_TILE(OP, 256, 128) \
    PCD_DECLARE_TILE(OP, 256, 256)
PCD_DECLARE_OP(float)
PCD_DECLARE_OP(bf16_t)
PCD_DECLARE_OP(f16_t)
extern template hipError_t launch_phase_tile<bf16_t, 64, 128, true>(int, const ProblemSet&, const PhaseArgs&, int,
                                                                    hipStream_t);
extern template hipError_t launch_phase_tile<f16_t, 64, 128, true>(int, const ProblemSet&, const PhaseArgs&, int,
                                                                   hipStream_t);
#undef PCD_DECLARE_OP
#undef PCD_DECLARE_TILE

}  // namespace pcd
