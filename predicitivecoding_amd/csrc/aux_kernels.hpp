// aux_kernels.hpp -- the small kernels around the phase GEMMs: zero fill,
// operand packing and the ragged early-exit decision.  Included by the host
// translation unit only (each definition here must exist once in the library).
#pragma once
#include "pc_kernels.hpp"

namespace pcd {


// Zero-fill of n 16-byte units (used inside captured graphs instead of
// hipMemsetAsync).
__global__ void zero_kernel(u32x4* __restrict__ p, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) p[i] = u32x4{0u, 0u, 0u, 0u};
}

// Pack a row-major [rows x cols] fp32 matrix (optionally read transposed) into
// a zero-padded [prow x pcol] buffer of the operand type whose rows are `ldd`
// elements apart (ldd >= pcol; the columns past pcol are left alone).
template <typename OP>
__global__ void pack_kernel(const void* __restrict__ src, int src_is_f32, int rows, int cols, int trans,
                            void* __restrict__ dst, int prow, int pcol, int ldd) {
    size_t n = (size_t)prow * pcol;
    for (size_t k = (size_t)blockIdx.x * blockDim.x + threadIdx.x; k < n; k += (size_t)gridDim.x * blockDim.x) {
        int r = (int)(k / pcol), c = (int)(k % pcol);
        const size_t i = (size_t)r * ldd + c;
        float v = 0.f;
        bool inside = r < rows && c < cols;
        if (inside) {
            // logical element (r, c) of op(src); physical src is [rows x cols] or [cols x rows]
            size_t s = trans ? (size_t)c * rows + r : (size_t)r * cols + c;
            if (src_is_f32) {
                v = ((const float*)src)[s];
            } else {
                // 16-bit source of the operand's own type: copy the bits
                ((uint16_t*)dst)[i] = ((const uint16_t*)src)[s];
                continue;
            }
        }
        if (!inside && !src_is_f32) { ((uint16_t*)dst)[i] = 0; continue; }
        OpTraits<OP>::store(dst, i, v);
    }
}

// Ragged early exit, one workgroup per request, between the error and the
// update phase of step t: sums the request's row energies, records them and
// decides whether step t is its last (Network.cs:895-905).
__global__ void exit_kernel(const float* __restrict__ part, int ldp, int nslots, const int* __restrict__ row_offsets,
                            int* __restrict__ done_at, float* __restrict__ prev_energy, float* __restrict__ last_energy,
                            int t, int rule, float thr) {
    const int r = blockIdx.x;
    if (t >= done_at[r]) return;  // uniform over the workgroup
    const int r0 = row_offsets[r], r1 = row_offsets[r + 1];
    float s = 0.f;
    for (int row = r0 + threadIdx.x; row < r1; row += blockDim.x)
        for (int k = 0; k < nslots; ++k) s += part[(size_t)k * ldp + row];
    __shared__ float red[256];
    red[threadIdx.x] = s;
    __syncthreads();
    for (int w = blockDim.x / 2; w > 0; w >>= 1) {
        if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const float e = red[0];
        const float prev = prev_energy[r];
        bool stop = false;
        if (rule == 1) stop = thr > 0.f && t > 0 && (prev - e < thr * fmaxf(prev, 1e-12f));
        else if (rule == 2) stop = e / (float)(r1 - r0) < thr;
        last_energy[r] = e;
        prev_energy[r] = e;
        if (stop) done_at[r] = t + 1;
    }
}

}  // namespace pcd
