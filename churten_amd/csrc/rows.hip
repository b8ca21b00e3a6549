// rows.hip -- replica-row transfers between (R, ...) device buffers and host
// mirrors, for the ensemble snapshot / checkpoint path.
//
// The reference's `Snapshot.update` (src/torchstrap/callbacks/training.py:
// 45-85) gathers the improved replicas' rows of every state leaf on the device,
// copies them into a pinned staging buffer of the whole state's size, syncs,
// and scatters them on the host into a pageable mirror. Here the mirror itself
// is pinned, and each leaf's selected rows are moved by the DMA engines
// straight between the live buffer and the mirror: one copy per run of
// consecutive selected rows (a plain copy when both sides are row-contiguous,
// a pitched 2-D copy otherwise). Nothing is gathered or staged, no kernel runs,
// nothing is synchronised.

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "../../include/churten_optim.h"

extern "C" int ts_copy_rows(void* dst, int64_t dst_stride, const void* src, int64_t src_stride,
                            int64_t row_bytes, const uint8_t* rows, int64_t R, int direction,
                            void* stream) {
  hipMemcpyKind kind;
  switch (direction) {
    case TS_ROWS_TO_HOST: kind = hipMemcpyDeviceToHost; break;
    case TS_ROWS_TO_DEVICE: kind = hipMemcpyHostToDevice; break;
    case TS_ROWS_DEVICE: kind = hipMemcpyDeviceToDevice; break;
    default: return static_cast<int>(hipErrorInvalidValue);
  }
  if (R < 0 || row_bytes < 0 || dst_stride < row_bytes || src_stride < row_bytes) {
    return static_cast<int>(hipErrorInvalidValue);
  }
  if (R == 0 || row_bytes == 0) return 0;
  if (dst == nullptr || src == nullptr) return static_cast<int>(hipErrorInvalidValue);
  const auto s = static_cast<hipStream_t>(stream);
  auto* d = static_cast<char*>(dst);
  const auto* sp = static_cast<const char*>(src);
  const bool packed = dst_stride == row_bytes && src_stride == row_bytes;
  int64_t r = 0;
  while (r < R) {
    if (rows != nullptr && rows[r] == 0) {
      ++r;
      continue;
    }
    int64_t end = r + 1;
    while (end < R && (rows == nullptr || rows[end] != 0)) ++end;
    const int64_t n = end - r;
    hipError_t err;
    if (packed) {
      err = hipMemcpyAsync(d + r * dst_stride, sp + r * src_stride,
                           static_cast<size_t>(n * row_bytes), kind, s);
    } else {
      err = hipMemcpy2DAsync(d + r * dst_stride, static_cast<size_t>(dst_stride),
                             sp + r * src_stride, static_cast<size_t>(src_stride),
                             static_cast<size_t>(row_bytes), static_cast<size_t>(n), kind, s);
    }
    if (err != hipSuccess) return static_cast<int>(err);
    r = end;
  }
  return 0;
}
