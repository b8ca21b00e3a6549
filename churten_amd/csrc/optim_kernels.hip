// optim_kernels.hip -- the extern "C" entry points of include/churten_optim.h
// that no single optimizer owns: the version, the workspace size, the steps
// bump and the gradient scatter. The optimizers' entry points are in
// abi_adam.hip, abi_sgd.hip and abi_adagrad.hip (the kernels, their launch
// shapes and the argument checks are in optim_drivers.h).

#include <hip/hip_runtime.h>

#include <stdint.h>

#include <algorithm>

#include "optim_dispatch.h"

namespace churten {
namespace {

// Copies every segment into its columns of the (R, cols) buffer `dst`.
template <typename T>
int scatter(const ts_segment* segs, int n_segs, void* dst, int64_t dst_stride_r, int64_t cols,
            int64_t R, hipStream_t stream) {
  if (R < 0 || cols < 0 || n_segs < 0 || (n_segs > 0 && segs == nullptr)) return kInvalid;
  if (!segments_valid(segs, n_segs, cols)) return kInvalid;
  if (R == 0) return 0;
  ScatterArgs<T> a;
  a.dst = static_cast<T*>(dst);
  a.dst_stride_r = dst_stride_r;
  constexpr uint32_t A = align_elems<T>();
  const bool vec_rows = reinterpret_cast<uintptr_t>(dst) % sizeof(T) == 0;
  a.res0 = static_cast<uint32_t>((reinterpret_cast<uintptr_t>(dst) / sizeof(T)) % A);
  a.rmod = static_cast<uint32_t>(((dst_stride_r % A) + A) % A);
  const SegmentWalk walk{segs, n_segs, cols, false};
  const bool any = std::any_of(segs, segs + n_segs, [](const ts_segment& s) {
    return s.numel > 0;
  });
  if ((any && dst == nullptr) ||
      !walk_fits<T>(walk, R, scatter_tile<T>(), vec_rows, a.seg, kScatterThreads)) {
    return kInvalid;
  }
  return launch_walk<T>(walk, R, scatter_tile<T>(), vec_rows, a, a.seg, scatter_kernel<T>, stream,
                        kScatterLds, kScatterThreads);
}

}  // namespace
}  // namespace churten

using churten::by_dtype;

extern "C" {

int ts_version(void) { return 200; }

size_t ts_workspace_bytes(int64_t R) {
  return R > 0 ? static_cast<size_t>(R) * churten::kPreStride * sizeof(double) : 0;
}

int ts_bump_steps(ts_dtype dtype, void* state_steps, const uint8_t* active_mask,
                  int64_t R, void* out_zero, void* stream) {
  if (R < 0 || (R > 0 && (state_steps == nullptr || active_mask == nullptr))) {
    return churten::kInvalid;
  }
  return by_dtype(dtype, [&](auto param) {
    using T = typename decltype(param)::type;
    return churten::launch_bump<T>(state_steps, active_mask, R, out_zero,
                                   static_cast<hipStream_t>(stream));
  });
}

int ts_scatter_segments(const ts_segment* src, int n_src, ts_dtype dtype, void* dst,
                        int64_t dst_stride_r, int64_t cols, int64_t R, void* stream) {
  return by_dtype(dtype, [&](auto param) {
    using T = typename decltype(param)::type;
    return churten::scatter<T>(src, n_src, dst, dst_stride_r, cols, R,
                               static_cast<hipStream_t>(stream));
  });
}

}  // extern "C"
