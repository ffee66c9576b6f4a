// gqa_rope.hip -- rotate_half RoPE on BF16 rows (the rope_unit of rope_unit.v:38-330,
// computed in double with closed-form angles as pyfiles/gen_gqa_wrapper_vectors.py:25-35
// does, then rounded double -> f32 -> BF16 as pyfiles/gqa_reference.py:15-19 does).
//
// One wave per row: lane i rotates the pair (i, i+64).
#include "gqa_device.h"
#include "gqa_internal.h"

namespace gqa {

__global__ __launch_bounds__(256) void rope_rows_kernel(RopeArgs a) {
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int i = threadIdx.x & 63;
    if (row >= a.n_rows) return;
    const int64_t pos = a.positions ? static_cast<int64_t>(a.positions[row])
                                    : static_cast<int64_t>(a.pos0) + row;
    const uint16_t* src = a.in + row * a.row_stride;
    uint16_t* dst = a.out + row * a.row_stride;
    double xr, yr;
    rope_pair(bf16_to_f32(src[i]), bf16_to_f32(src[i + kPairs]), pos, a.rope.inv_freq[i], xr, yr);
    dst[i] = f64_to_bf16_via_f32(xr);
    dst[i + kPairs] = f64_to_bf16_via_f32(yr);
}

hipError_t launch_rope_rows(const RopeArgs& a, hipStream_t stream) {
    const int64_t blocks = (a.n_rows + 3) / 4;
    hipLaunchKernelGGL(rope_rows_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace gqa
