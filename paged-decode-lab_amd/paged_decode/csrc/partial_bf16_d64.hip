// Partition kernels for BF16 q (BF16 or FP8 K/V, matrix-core kernel), head_dim 64: one translation unit of
// the gfx950 decode library (see partition_kernels.h).
#include "partition_kernels.h"

namespace pd {

int dispatch_partial_bf16_d64(PartialParams& prm, int kv_dtype, int kv_heads, hipStream_t stream) {
    return dispatch_kv<__bf16, 64>(prm, kv_dtype, kv_heads, stream);
}

}  // namespace pd
