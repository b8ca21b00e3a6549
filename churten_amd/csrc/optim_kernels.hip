// optim_kernels.hip -- the extern "C" entry points of include/churten_optim.h:
// the dispatch of each call onto the policy its flags and dtype select (the
// kernels, their launch shapes and the argument checks are in
// optim_drivers.h), and the allocation-free form's device scratch.

#include <hip/hip_runtime.h>

#include <stdint.h>

#include <mutex>

#include "../../include/churten_optim.h"
#include "optim_drivers.h"

namespace churten {
namespace {

// Runs `launch` with the policy that matches the call's flags and the number
// of (R, T) operands that policy reads.
template <typename T, typename S, typename Launch>
int adam_dispatch(uint32_t flags, Launch&& launch) {
  const bool amsgrad = (flags & TS_AMSGRAD) != 0;
  const bool adamw = (flags & TS_ADAMW) != 0;
  if (adamw) {
    if (amsgrad) return launch(AdamPolicy<T, true, true, S>{}, 5);
    return launch(AdamPolicy<T, true, false, S>{}, 4);
  }
  if (amsgrad) return launch(AdamPolicy<T, false, true, S>{}, 5);
  return launch(AdamPolicy<T, false, false, S>{}, 4);
}

template <typename T, typename S, typename Launch>
int sgd_dispatch(uint32_t flags, bool has_buf, bool work, Launch&& launch) {
  const bool nesterov = (flags & TS_NESTEROV) != 0;
  if (has_buf) {
    if (nesterov) return launch(SgdPolicy<T, true, true, S>{}, 3);
    return launch(SgdPolicy<T, true, false, S>{}, 3);
  }
  // Nesterov needs momentum buffers -- when there is an element to update: an
  // empty (R, T) buffer may come with a NULL data pointer, and a call with R
  // or T of 0 only bumps the steps, as the reference's does.
  if (nesterov && work) return kInvalid;
  return launch(SgdPolicy<T, false, false, S>{}, 2);
}

template <typename T, typename S, typename Launch>
int adagrad_dispatch(uint32_t flags, Launch&& launch) {
  if ((flags & TS_ADAGRAD_F32) != 0) {
    if constexpr (std::is_same<T, double>::value) {
      return kInvalid;
    } else {
      return launch(AdagradF32Policy<T, S>{}, 3);
    }
  }
  return launch(AdagradPolicy<T, S>{}, 3);
}

template <typename U>
struct type_tag {
  using type = U;
};

// The optimizer-state type of a call: the parameter type, or bfloat16 under
// TS_STATE_BF16 (float32 parameters only).
template <typename T, typename Launch>
int with_state_type(uint32_t flags, Launch&& launch) {
  if ((flags & TS_STATE_BF16) == 0) return launch(type_tag<T>{});
  if constexpr (std::is_same<T, float>::value) {
    return launch(type_tag<bf16_t>{});
  } else {
    return kInvalid;
  }
}

template <template <typename> class Body, typename... Args>
int by_dtype(ts_dtype dtype, Args&&... args) {
  switch (dtype) {
    case TS_FLOAT32: return Body<float>::run(args...);
    case TS_FLOAT64: return Body<double>::run(args...);
    case TS_FLOAT16: return Body<_Float16>::run(args...);
    case TS_BFLOAT16: return Body<bf16_t>::run(args...);
  }
  return kInvalid;
}

template <typename P>
int launch_any(const Call& c, int nbufs, const ts_segment* segs, int n_segs, bool segmented) {
  return segmented ? launch_segments<P>(c, nbufs, segs, n_segs) : launch_dense<P>(c, nbufs);
}

template <typename T>
struct AdamBody {
  static int run(const Call& c, const ts_segment* segs, int n_segs, bool segmented) {
    return with_state_type<T>(c.flags, [&](auto state) {
      using S = typename decltype(state)::type;
      return adam_dispatch<T, S>(c.flags, [&](auto policy, int nbufs) {
        return launch_any<decltype(policy)>(c, nbufs, segs, n_segs, segmented);
      });
    });
  }
};

template <typename T>
struct SgdBody {
  static int run(const Call& c, const ts_segment* segs, int n_segs, bool segmented) {
    const bool has_buf = c.bufs != nullptr && c.bufs[2].data != nullptr;
    const bool work = c.R > 0 && c.T > 0;
    return with_state_type<T>(c.flags, [&](auto state) {
      using S = typename decltype(state)::type;
      return sgd_dispatch<T, S>(c.flags, has_buf, work, [&](auto policy, int nbufs) {
        return launch_any<decltype(policy)>(c, nbufs, segs, n_segs, segmented);
      });
    });
  }
};

template <typename T>
struct AdagradBody {
  static int run(const Call& c, const ts_segment* segs, int n_segs, bool segmented) {
    return with_state_type<T>(c.flags, [&](auto state) {
      using S = typename decltype(state)::type;
      return adagrad_dispatch<T, S>(c.flags, [&](auto policy, int nbufs) {
        return launch_any<decltype(policy)>(c, nbufs, segs, n_segs, segmented);
      });
    });
  }
};

template <typename T>
struct ScatterBody {
  static int run(const ts_segment* segs, int n_segs, void* dst, int64_t dst_stride_r,
                 int64_t cols, int64_t R, hipStream_t stream) {
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
    if ((any && dst == nullptr) || !walk_fits<T>(walk, R, kTile, vec_rows, a.seg)) return kInvalid;
    return launch_walk<T>(walk, R, kTile, vec_rows, a, a.seg, scatter_kernel<T>, stream);
  }
};

template <typename T>
struct BumpBody {
  static int run(void* steps, const uint8_t* mask, int64_t R, void* out_zero,
                 hipStream_t stream) {
    return launch_bump<T>(steps, mask, R, out_zero, stream);
  }
};


// Replicas whose per-replica constants fit ts_adam_step_noalloc's scratch.
constexpr int64_t kScratchReplicas = 65536;
constexpr int kMaxDevices = 64;

}  // namespace
}  // namespace churten

// The per-replica constants of ts_adam_step_noalloc (kPreStride doubles for up
// to kScratchReplicas replicas: 1 MiB), one copy on every device the library
// runs on, held until the process ends. In host code this name is only a
// stand-in: its device address comes from hipGetSymbolAddress
// (scratch_on_current_device), once per device.
static __device__ __align__(256) double scratch[churten::kPreStride * churten::kScratchReplicas];

namespace churten {
namespace {

// The device address of `scratch` on the calling thread's current device,
// looked up the first time the entry point runs on that device (with it
// current) and kept per device.
int scratch_on_current_device(void** out) {
  int dev = -1;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (dev < 0 || dev >= kMaxDevices) return kInvalid;
  static std::mutex mu;
  static void* addr[kMaxDevices] = {};
  const std::lock_guard<std::mutex> lock(mu);
  if (addr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t s = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (s != hipSuccess) return static_cast<int>(s);
    if (p == nullptr) return kInvalid;
    addr[dev] = p;
  }
  *out = addr[dev];
  return 0;
}

}  // namespace
}  // namespace churten

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
using churten::by_dtype;
using churten::make_call;

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
  return by_dtype<churten::BumpBody>(dtype, state_steps, active_mask, R, out_zero,
                                     static_cast<hipStream_t>(stream));
}

int ts_adam_step(const ts_rt_buf* bufs, ts_dtype dtype, void* state_steps,
                 const void* lr, const void* beta1, const void* beta2,
                 const void* eps, const void* weight_decay,
                 const uint8_t* active_mask, int64_t R, int64_t T,
                 uint32_t flags, void* out_zero, void* stream) {
  const auto c = make_call(bufs, state_steps, {lr, beta1, beta2, eps, weight_decay},
                           active_mask, R, T, flags, out_zero, stream);
  return by_dtype<churten::AdamBody>(dtype, c, nullptr, 0, false);
}

int ts_sgd_step(const ts_rt_buf* bufs, ts_dtype dtype, void* state_steps,
                const void* lr, const void* momentum, const void* dampening,
                const void* weight_decay, const uint8_t* active_mask,
                int64_t R, int64_t T, uint32_t flags, void* out_zero,
                void* stream) {
  const auto c = make_call(bufs, state_steps, {lr, momentum, dampening, weight_decay},
                           active_mask, R, T, flags, out_zero, stream);
  return by_dtype<churten::SgdBody>(dtype, c, nullptr, 0, false);
}

int ts_adagrad_step(const ts_rt_buf* bufs, ts_dtype dtype, void* state_steps,
                    const void* lr, const void* lr_decay,
                    const void* weight_decay, const void* eps,
                    const uint8_t* active_mask, int64_t R, int64_t T,
                    uint32_t flags, void* out_zero, void* stream) {
  const auto c = make_call(bufs, state_steps, {lr, lr_decay, weight_decay, eps},
                           active_mask, R, T, flags, out_zero, stream);
  return by_dtype<churten::AdagradBody>(dtype, c, nullptr, 0, false);
}

int ts_adam_step_segments(const ts_rt_buf* bufs, const ts_segment* grads, int n_grads,
                          ts_dtype dtype, void* state_steps, const void* lr,
                          const void* beta1, const void* beta2, const void* eps,
                          const void* weight_decay, const uint8_t* active_mask,
                          int64_t R, int64_t T, uint32_t flags, void* out_zero,
                          void* stream) {
  const auto c = make_call(bufs, state_steps, {lr, beta1, beta2, eps, weight_decay},
                           active_mask, R, T, flags, out_zero, stream);
  return by_dtype<churten::AdamBody>(dtype, c, grads, n_grads, true);
}

int ts_sgd_step_segments(const ts_rt_buf* bufs, const ts_segment* grads, int n_grads,
                         ts_dtype dtype, void* state_steps, const void* lr,
                         const void* momentum, const void* dampening,
                         const void* weight_decay, const uint8_t* active_mask,
                         int64_t R, int64_t T, uint32_t flags, void* out_zero,
                         void* stream) {
  const auto c = make_call(bufs, state_steps, {lr, momentum, dampening, weight_decay},
                           active_mask, R, T, flags, out_zero, stream);
  return by_dtype<churten::SgdBody>(dtype, c, grads, n_grads, true);
}

int ts_adagrad_step_segments(const ts_rt_buf* bufs, const ts_segment* grads, int n_grads,
                             ts_dtype dtype, void* state_steps, const void* lr,
                             const void* lr_decay, const void* weight_decay,
                             const void* eps, const uint8_t* active_mask, int64_t R,
                             int64_t T, uint32_t flags, void* out_zero, void* stream) {
  const auto c = make_call(bufs, state_steps, {lr, lr_decay, weight_decay, eps},
                           active_mask, R, T, flags, out_zero, stream);
  return by_dtype<churten::AdagradBody>(dtype, c, grads, n_grads, true);
}

int ts_adam_step_ws(const ts_rt_buf* bufs, ts_dtype dtype, void* state_steps, const void* lr,
                    const void* beta1, const void* beta2, const void* eps,
                    const void* weight_decay, const uint8_t* active_mask, int64_t R, int64_t T,
                    uint32_t flags, void* out_zero, void* workspace, size_t workspace_bytes,
                    void* stream) {
  if (workspace == nullptr) return churten::kInvalid;
  const auto c = make_call(bufs, state_steps, {lr, beta1, beta2, eps, weight_decay},
                           active_mask, R, T, flags, out_zero, stream, workspace,
                           workspace_bytes);
  return by_dtype<churten::AdamBody>(dtype, c, nullptr, 0, false);
}

int ts_adagrad_step_ws(const ts_rt_buf* bufs, ts_dtype dtype, void* state_steps,
                       const void* lr, const void* lr_decay, const void* weight_decay,
                       const void* eps, const uint8_t* active_mask, int64_t R, int64_t T,
                       uint32_t flags, void* out_zero, void* workspace, size_t workspace_bytes,
                       void* stream) {
  if (workspace == nullptr) return churten::kInvalid;
  const auto c = make_call(bufs, state_steps, {lr, lr_decay, weight_decay, eps}, active_mask,
                           R, T, flags, out_zero, stream, workspace, workspace_bytes);
  return by_dtype<churten::AdagradBody>(dtype, c, nullptr, 0, false);
}

int ts_adam_step_segments_ws(const ts_rt_buf* bufs, const ts_segment* grads, int n_grads,
                             ts_dtype dtype, void* state_steps, const void* lr,
                             const void* beta1, const void* beta2, const void* eps,
                             const void* weight_decay, const uint8_t* active_mask, int64_t R,
                             int64_t T, uint32_t flags, void* out_zero, void* workspace,
                             size_t workspace_bytes, void* stream) {
  if (workspace == nullptr) return churten::kInvalid;
  const auto c = make_call(bufs, state_steps, {lr, beta1, beta2, eps, weight_decay},
                           active_mask, R, T, flags, out_zero, stream, workspace,
                           workspace_bytes);
  return by_dtype<churten::AdamBody>(dtype, c, grads, n_grads, true);
}

int ts_adagrad_step_segments_ws(const ts_rt_buf* bufs, const ts_segment* grads, int n_grads,
                                ts_dtype dtype, void* state_steps, const void* lr,
                                const void* lr_decay, const void* weight_decay,
                                const void* eps, const uint8_t* active_mask, int64_t R,
                                int64_t T, uint32_t flags, void* out_zero, void* workspace,
                                size_t workspace_bytes, void* stream) {
  if (workspace == nullptr) return churten::kInvalid;
  const auto c = make_call(bufs, state_steps, {lr, lr_decay, weight_decay, eps}, active_mask,
                           R, T, flags, out_zero, stream, workspace, workspace_bytes);
  return by_dtype<churten::AdagradBody>(dtype, c, grads, n_grads, true);
}

int ts_adam_step_noalloc(const ts_rt_buf* bufs, ts_dtype dtype, void* state_steps,
                         const void* lr, const void* beta1, const void* beta2, const void* eps,
                         const void* weight_decay, const uint8_t* active_mask, int64_t R,
                         int64_t T, uint32_t flags, void* out_zero, void* stream) {
  if (R < 0 || R > churten::kScratchReplicas) return churten::kInvalid;
  void* ws = nullptr;
  const int err = churten::scratch_on_current_device(&ws);
  if (err != 0) return err;
  const auto c = make_call(bufs, state_steps, {lr, beta1, beta2, eps, weight_decay},
                           active_mask, R, T, flags, out_zero, stream, ws,
                           sizeof(double) * churten::kPreStride * churten::kScratchReplicas);
  return by_dtype<churten::AdamBody>(dtype, c, nullptr, 0, false);
}

int ts_scatter_segments(const ts_segment* src, int n_src, ts_dtype dtype, void* dst,
                        int64_t dst_stride_r, int64_t cols, int64_t R, void* stream) {
  return by_dtype<churten::ScatterBody>(dtype, src, n_src, dst, dst_stride_r, cols, R,
                                        static_cast<hipStream_t>(stream));
}

}  // extern "C"
