// optim_dispatch.h -- the dispatch of a C-ABI call onto the policy its dtype
// and flags select, shared by the entry-point translation units
// (abi_adam.hip, abi_adam_segments.hip, abi_sgd.hip, abi_adagrad.hip): each
// instantiates only the policies and driver families of its own entry points,
// so they compile in parallel. Like optim_drivers.h, everything is in an
// anonymous namespace.
#pragma once

#include <hip/hip_runtime.h>

#include <stdint.h>

#include <type_traits>

#include "../../include/churten_optim.h"
#include "optim_drivers.h"

namespace churten {
namespace {

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

// Calls `f` with the type_tag of the parameter type `dtype` names.
template <typename F>
int by_dtype(ts_dtype dtype, F&& f) {
  switch (dtype) {
    case TS_FLOAT32: return f(type_tag<float>{});
    case TS_FLOAT64: return f(type_tag<double>{});
    case TS_FLOAT16: return f(type_tag<_Float16>{});
    case TS_BFLOAT16: return f(type_tag<bf16_t>{});
  }
  return kInvalid;
}

// The dense driver families (launch_dense) or the segmented one
// (launch_segments): a translation unit instantiates only the one it calls.
template <typename P, bool SEGMENTED>
int launch_any(const Call& c, int nbufs, const ts_segment* segs, int n_segs) {
  if constexpr (SEGMENTED) {
    return launch_segments<P>(c, nbufs, segs, n_segs);
  } else {
    return launch_dense<P>(c, nbufs);
  }
}

// Runs `launch` with the Adam policy that matches the call's flags and the
// number of (R, T) operands that policy reads.
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

// One optimizer step of the call: parameter type, state type, then the
// optimizer's flags select the policy.
template <bool SEGMENTED>
int adam_run(ts_dtype dtype, const Call& c, const ts_segment* segs, int n_segs) {
  return by_dtype(dtype, [&](auto param) {
    using T = typename decltype(param)::type;
    return with_state_type<T>(c.flags, [&](auto state) {
      using S = typename decltype(state)::type;
      return adam_dispatch<T, S>(c.flags, [&](auto policy, int nbufs) {
        return launch_any<decltype(policy), SEGMENTED>(c, nbufs, segs, n_segs);
      });
    });
  });
}

template <bool SEGMENTED>
int sgd_run(ts_dtype dtype, const Call& c, const ts_segment* segs, int n_segs) {
  const bool has_buf = c.bufs != nullptr && c.bufs[2].data != nullptr;
  const bool work = c.R > 0 && c.T > 0;
  return by_dtype(dtype, [&](auto param) {
    using T = typename decltype(param)::type;
    return with_state_type<T>(c.flags, [&](auto state) {
      using S = typename decltype(state)::type;
      return sgd_dispatch<T, S>(c.flags, has_buf, work, [&](auto policy, int nbufs) {
        return launch_any<decltype(policy), SEGMENTED>(c, nbufs, segs, n_segs);
      });
    });
  });
}

template <bool SEGMENTED>
int adagrad_run(ts_dtype dtype, const Call& c, const ts_segment* segs, int n_segs) {
  return by_dtype(dtype, [&](auto param) {
    using T = typename decltype(param)::type;
    return with_state_type<T>(c.flags, [&](auto state) {
      using S = typename decltype(state)::type;
      return adagrad_dispatch<T, S>(c.flags, [&](auto policy, int nbufs) {
        return launch_any<decltype(policy), SEGMENTED>(c, nbufs, segs, n_segs);
      });
    });
  });
}

}  // namespace
}  // namespace churten
