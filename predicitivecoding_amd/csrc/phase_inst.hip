// phase_inst.hip -- one (operand type, tile) instantiation of the phase kernels.
//
// Compiled once per combination with
//   -DPCD_OP_ID=0|1|2   (fp32, bf16, fp16 operands)
//   -DPCD_BM=64|128|256 -DPCD_BN=64|128|256
//   -DPCD_WD=1          (the direct-weight 64 x 128 tile of the 16-bit types)
// and linked into libpcdevice_hip.so next to pcdevice.hip.
#include "phase_launch.hpp"

#if !defined(PCD_OP_ID) || !defined(PCD_BM) || !defined(PCD_BN)
#error "phase_inst.hip needs PCD_OP_ID, PCD_BM and PCD_BN"
#endif
#ifndef PCD_WD
#define PCD_WD 0   // 1: the direct-weight form of the tile (16-bit 64 x 128 only)
#endif

namespace pcd {

#if PCD_OP_ID == 0
typedef float InstOp;
#elif PCD_OP_ID == 1
typedef bf16_t InstOp;
#else
typedef f16_t InstOp;
#endif

template <typename OP, int BM, int BN, bool WD>
hipError_t launch_phase_tile(int epi, const ProblemSet& set, const PhaseArgs& args, int grid, hipStream_t s) {
    const dim3 block(TileCfg<BM, BN, OpTraits<OP>::bytes, WD>::NT);
    switch (epi) {
    case EPI_ERROR: hipLaunchKernelGGL((phase_kernel<OP, BM, BN, EPI_ERROR, WD>), dim3(grid), block, 0, s, set, args); break;
    case EPI_UPDATE: hipLaunchKernelGGL((phase_kernel<OP, BM, BN, EPI_UPDATE, WD>), dim3(grid), block, 0, s, set, args); break;
    case EPI_FFG: hipLaunchKernelGGL((phase_kernel<OP, BM, BN, EPI_FFG, WD>), dim3(grid), block, 0, s, set, args); break;
    case EPI_PLAIN_KN:
    case EPI_PLAIN_MK:
    case EPI_PLAIN_MKKN:
        if constexpr (kn_tile(OpTraits<OP>::bytes, BM, BN, WD)) {
            if (epi == EPI_PLAIN_KN)
                hipLaunchKernelGGL((phase_kernel<OP, BM, BN, EPI_PLAIN_KN, WD>), dim3(grid), block, 0, s, set, args);
            else if (epi == EPI_PLAIN_MK)
                hipLaunchKernelGGL((phase_kernel<OP, BM, BN, EPI_PLAIN_MK, WD>), dim3(grid), block, 0, s, set, args);
            else
                hipLaunchKernelGGL((phase_kernel<OP, BM, BN, EPI_PLAIN_MKKN, WD>), dim3(grid), block, 0, s, set, args);
            break;
        } else {
            return hipErrorInvalidValue;   // no transposed-operand form of this tile
        }
    default: hipLaunchKernelGGL((phase_kernel<OP, BM, BN, EPI_PLAIN, WD>), dim3(grid), block, 0, s, set, args); break;
    }
    return hipGetLastError();
}

template hipError_t launch_phase_tile<InstOp, PCD_BM, PCD_BN, (bool)PCD_WD>(int, const ProblemSet&, const PhaseArgs&,
                                                                           int, hipStream_t);

#if PCD_OP_ID == 0 && PCD_BM == 64 && PCD_BN == 64
template <typename OP, int BM, int BN>
hipError_t launch_persistent_tile(const PersistArgs& args, int grid, hipStream_t s) {
    void* params[] = {(void*)&args};
    return hipLaunchCooperativeKernel((const void*)persistent_relax_kernel<OP, BM, BN>, dim3(grid),
                                      dim3(TileCfg<BM, BN>::NT), params, 0, s);
}
template hipError_t launch_persistent_tile<float, 64, 64>(const PersistArgs&, int, hipStream_t);

int persistent_blocks_per_cu() {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, (const void*)persistent_relax_kernel<float, 64, 64>,
                                                     TileCfg<64, 64>::NT, 0) != hipSuccess)
        return 0;
    return n;
}
#endif

}  // namespace pcd
