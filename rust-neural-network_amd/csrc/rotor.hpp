// rotor.hpp -- Cl(3,0) rotor arithmetic of src/quant.rs shared by the
// RotorQuant kernels: the rotor product and the 3x3 rotation matrix, in the
// reference's expression order (every file is built without contraction).
#pragma once

#include <hip/hip_runtime.h>

namespace rnn {

// rotor * x on a multivector [1,e1,e2,e3,e12,e13,e23,e123] (src/quant.rs:70-81)
__device__ __forceinline__ void rotor_apply(const float *x, float s, float p12, float p13,
                                            float p23, float *o) {
    o[0] = s * x[0] - p12 * x[4] - p13 * x[5] - p23 * x[6];
    o[1] = s * x[1] + p12 * x[2] + p13 * x[3] + p23 * x[7];
    o[2] = s * x[2] - p12 * x[1] + p23 * x[3] - p13 * x[7];
    o[3] = s * x[3] - p13 * x[1] - p23 * x[2] + p12 * x[7];
    o[4] = s * x[4] + p12 * x[0];
    o[5] = s * x[5] + p13 * x[0];
    o[6] = s * x[6] + p23 * x[0];
    o[7] = s * x[7] - p23 * x[1] + p13 * x[2] - p12 * x[3];
}

// Rotor::rotation_matrix: column j is the vector part of R e_j R~
// (src/quant.rs:84-89, :101-113). rot is row-major 3x3.
__device__ __forceinline__ void rotation_matrix(const float *r, float *rot) {
    for (int j = 0; j < 3; ++j) {
        float e[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        e[1 + j] = 1.0f;
        float t[8], o[8];
        rotor_apply(e, r[0], r[1], r[2], r[3], t);
        rotor_apply(t, r[0], -r[1], -r[2], -r[3], o);
        rot[0 * 3 + j] = o[1];
        rot[1 * 3 + j] = o[2];
        rot[2 * 3 + j] = o[3];
    }
}

}  // namespace rnn
