// winograd_tf.h - the 1-D F(4x4,3x3) transforms shared by the three-launch and the
// fused Winograd kernels (Lavin & Gray 2015, "Fast Algorithms for Convolutional
// Neural Networks", interpolation points 0, 1, -1, 2, -2, inf). The 2-D transforms
// apply them to the columns first, then to the rows, in both kernels, so the two
// compute the same transform-domain values.
#pragma once
#include <hip/hip_runtime.h>

namespace spinn {

// 1-D transforms of F(4,3) (Lavin & Gray 2015, points 0, 1, -1, 2, -2, inf).
__device__ __forceinline__ void bt6(const float d[6], float o[6]) {   // B^T (6x6)
    o[0] = 4.f * d[0] - 5.f * d[2] + d[4];
    o[1] = -4.f * d[1] - 4.f * d[2] + d[3] + d[4];
    o[2] = 4.f * d[1] - 4.f * d[2] - d[3] + d[4];
    o[3] = -2.f * d[1] - d[2] + 2.f * d[3] + d[4];
    o[4] = 2.f * d[1] - d[2] - 2.f * d[3] + d[4];
    o[5] = 4.f * d[1] - 5.f * d[3] + d[5];
}

__device__ __forceinline__ void g6(const float g[3], float o[6]) {    // G (6x3)
    o[0] = 0.25f * g[0];
    o[1] = (g[0] + g[1] + g[2]) * (-1.f / 6.f);
    o[2] = (g[0] - g[1] + g[2]) * (-1.f / 6.f);
    o[3] = g[0] * (1.f / 24.f) + g[1] * (1.f / 12.f) + g[2] * (1.f / 6.f);
    o[4] = g[0] * (1.f / 24.f) - g[1] * (1.f / 12.f) + g[2] * (1.f / 6.f);
    o[5] = g[2];
}

__device__ __forceinline__ void at6(const float m[6], float o[4]) {   // A^T (4x6)
    const float p12 = m[1] + m[2], m12 = m[1] - m[2], p34 = m[3] + m[4], m34 = m[3] - m[4];
    o[0] = m[0] + p12 + p34;
    o[1] = m12 + 2.f * m34;
    o[2] = p12 + 4.f * p34;
    o[3] = m12 + 8.f * m34 + m[5];
}

} // namespace spinn
