// Launchers shared between the kernel translation units and the C-ABI layer.
// Every launcher validates its arguments on the host, enqueues on `stream`
// and returns a Status (0 on success); none of them synchronizes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace asmhip {

enum class QuantType { Q4_0, Q8_0 };

// y = W x.  gguf: W is [M][K/32] GGUF blocks; otherwise W is the split qs
// array and `scales` the fp32 [M][K/32] scales.
int matvec_launch(QuantType qt, bool gguf, const void* w, const float* scales, const float* x, float* y,
                  int64_t M, int64_t K, hipStream_t stream);

// Exact fp32 dequantization of GGUF blocks, row-major [rows][K].
int dequant_launch(QuantType qt, const void* w, float* out, int64_t rows, int64_t K, hipStream_t stream);

}  // namespace asmhip
