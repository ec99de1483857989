/* q8_gemm.hip: Y = X W^T for 5 <= t <= 64 tokens. */
#include <hip/hip_runtime.h>

#include "q8_device.h"

void q8_launch_gemm(q8_stream_t stream, const void *w0, const void *w1, long rows, long cols, const float *x, long x_stride, long t, float *y)
{
    q8_launch_gemv(stream, w0, w1, rows, cols, x, x_stride, t, y);
}
