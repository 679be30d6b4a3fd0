// The Medusa residual block's fc projections through the weight-streaming kernel of
// lm_head.hip (called by fg_medusa_heads, gemm.hip).
#pragma once

#include "fg_common.h"

namespace fg {

// bf16 shapes the stream runs: batch <= 256, H a multiple of 64, every head's weight and
// activation span below 4 GiB.
bool medusa_stream_ok(int batch, int H, int heads);
// fp32 partial sums the stream needs in the caller's workspace (0 when it cannot run).
size_t medusa_stream_parts_bytes(int batch, int H, int heads);
// out[h * batch + b, :] = R[b, :] + SiLU(a[h, b, :] . fc_w[h]^T + fc_b[h]) with a the
// normalised rows [heads, batch, H] (bf16), fc_w [heads, H, H], fc_b [heads, H] (bf16):
// the weight is streamed once in key ranges whose fp32 sums go to `parts`, then a second
// launch adds the ranges in order and applies bias, SiLU and the residual.
int medusa_stream(const void* a, int batch, int H, int heads, const void* fc_w, const void* fc_b, const void* R,
                  int64_t ldr, int r_dtype, void* out, int out_dtype, float* parts, hipStream_t s);

}  // namespace fg
