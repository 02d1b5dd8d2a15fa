// Partition kernels for FP32 q/K/V (vector-ALU kernel), head_dim 64: one translation unit of
// the gfx950 decode library (see partition_kernels.h).
#include "partition_kernels.h"

namespace pd {

int dispatch_partial_f32_d64(PartialParams& prm, int kv_dtype, int kv_heads, hipStream_t stream) {
    (void)kv_dtype;  // K/V share q's format
    return dispatch_fp32<64>(prm, kv_heads, stream);
}

}  // namespace pd
