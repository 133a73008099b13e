// Host launchers of the any-shape kernels (csrc/generic.hip) that the tuned entry points
// dispatch to for shapes or I/O types they do not cover.  Same argument meaning as the
// corresponding tops_tmu_* entry points; each returns a TOPS_* status.
#pragma once

#include "capi.hpp"

namespace tops {

int tmu_generic_input_phase(const void* x, const void* mask, const void* Wp, const void* Wg, const float* Bp,
                            const float* Bg, void* ab, int64_t B, int64_t L, int64_t C, int64_t C_out, int64_t ld,
                            int transpose, float eps, int dtype, hipStream_t st);
int tmu_generic_output_phase(const void* y, const void* x, const void* Wp, const void* Wg, const float* Bp,
                             const float* Bg, const void* res, void* out, int64_t B, int64_t L, int64_t C,
                             int64_t C_out, int64_t ldy, float eps, int dtype, hipStream_t st);

}  // namespace tops
