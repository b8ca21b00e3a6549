// optim_kernels.hip -- gfx950 kernels and the extern "C" launchers of
// include/churten_optim.h.
//
// Work decomposition. The consolidated (R, T) state is cut into tiles of
// kTile = kThreads * kPack * kUnroll consecutive elements of one row; the 1-D
// grid enumerates (replica, tile) pairs replica-major, so blockIdx.x alone
// gives both and no grid dimension caps R. A workgroup first reads its
// replica's active flag: a frozen replica is a workgroup-uniform early exit, so
// its rows are never read or written (they stay bit-identical, and a replica
// frozen at step 0 never evaluates 1 - beta^0 = 0). Active workgroups read the
// replica's hyperparameters once (scalar loads: the address is uniform), derive
// the per-replica constants, then stream their tile.
//
// Streaming path (unit inner stride, T % 4 == 0, 16-byte aligned rows, which is
// the layout the consolidation produces): every thread issues kUnroll 16-byte
// non-temporal loads per buffer before any arithmetic, then computes and issues
// the non-temporal stores.
// Element path (any strides, ragged T): the same tile geometry with one element
// per access; the per-element arithmetic is the same inlined function, so both
// paths give bit-identical results for the same element.
//
// Everything is enqueued on the caller's stream; nothing is allocated.

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "../../include/churten_optim.h"
#include "optim_math.h"

namespace churten {
namespace {

// Launch shape, measured on the MI355X over the 52 GB north-star state: 128
// threads x 2 packs of 4 elements per thread (1024-element tiles) with
// non-temporal vector loads and stores gave the best HBM throughput of the
// shapes tried (64..1024 threads, 1..8 packs, persistent grid-stride loops,
// XCD-contiguous tile order); non-temporal hints on both loads and stores were
// worth ~10% over plain accesses, either alone nothing.
constexpr int kThreads = 128;
constexpr int kPack = 4;
constexpr int kUnroll = 2;
constexpr int64_t kTile = int64_t(kThreads) * kPack * kUnroll;

template <typename T>
struct alignas(sizeof(T) * kPack) Pack {
  T v[kPack];
};

// A pack as raw 32-bit words, so it can go through the non-temporal builtins
// (16 B for fp32, 8 B for 16-bit types, 32 B for fp64).
template <typename T>
using PackBits = uint32_t __attribute__((ext_vector_type(sizeof(T) * kPack / 4)));

// Streaming accesses: every byte of the optimizer state is touched exactly
// once per step, so the loads and stores carry the non-temporal hint.
template <typename T>
__device__ __forceinline__ Pack<T> load_stream(const Pack<T>* p) {
  return __builtin_bit_cast(
      Pack<T>, __builtin_nontemporal_load(reinterpret_cast<const PackBits<T>*>(p)));
}

template <typename T>
__device__ __forceinline__ void store_stream(Pack<T>* p, const Pack<T>& v) {
  __builtin_nontemporal_store(__builtin_bit_cast(PackBits<T>, v),
                              reinterpret_cast<PackBits<T>*>(p));
}

// Up to five (R, T) operands. `data[i]` is element (0, 0) of operand i.
template <typename T>
struct Operands {
  T* data[5];
  int64_t stride_r[5];
  int64_t stride_t[5];
};

struct Grid {
  int64_t T;
  uint32_t tiles_per_row;
};

__device__ __forceinline__ void tile_of_block(const Grid& g, uint32_t& r,
                                              int64_t& t0) {
  const uint32_t tile = blockIdx.x;
  r = tile / g.tiles_per_row;
  t0 = int64_t(tile - r * g.tiles_per_row) * kTile;
}

// ---------------------------------------------------------------------------
// state_steps += active_mask, and the zero return scalar.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(kThreads) void bump_steps_kernel(
    T* __restrict__ steps, const uint8_t* __restrict__ mask, int64_t R,
    T* __restrict__ out_zero) {
  const int64_t r = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (r < R) {
    const op_t<T> one = mask[r] ? op_t<T>(1) : op_t<T>(0);
    steps[r] = narrow<T>(widen(steps[r]) + one);
  }
  if (out_zero != nullptr && r == 0) {
    *out_zero = narrow<T>(op_t<T>(0));
  }
}

// ---------------------------------------------------------------------------
// Adam / AdamW
// ---------------------------------------------------------------------------
template <typename T>
struct AdamArgs {
  Operands<T> x;  // param, grad, exp_avg, exp_avg_sq, max_exp_avg_sq
  const T* steps;
  const T* lr;
  const T* beta1;
  const T* beta2;
  const T* eps;
  const T* weight_decay;
  const uint8_t* mask;
  Grid g;
  bool maximize;
};

template <typename T>
__device__ __forceinline__ bool adam_prologue(const AdamArgs<T>& a, uint32_t r,
                                              AdamHyper& h, op_t<T>& bc1,
                                              op_t<T>& bc2s) {
  if (!a.mask[r]) {
    return false;
  }
  h.lr = static_cast<double>(widen(a.lr[r]));
  h.beta1 = static_cast<double>(widen(a.beta1[r]));
  h.beta2 = static_cast<double>(widen(a.beta2[r]));
  h.weight_decay = static_cast<double>(widen(a.weight_decay[r]));
  h.eps = static_cast<double>(widen(a.eps[r]));
  adam_bias_corrections<op_t<T>>(h.beta1, h.beta2,
                                 static_cast<double>(widen(a.steps[r])), bc1,
                                 bc2s);
  return true;
}

template <typename T, bool ADAMW, bool AMSGRAD>
__global__ __launch_bounds__(kThreads) void adam_stream_kernel(AdamArgs<T> a) {
  using opmath_t = op_t<T>;
  constexpr int NB = AMSGRAD ? 5 : 4;
  uint32_t r;
  int64_t t0;
  tile_of_block(a.g, r, t0);
  AdamHyper h;
  opmath_t bc1, bc2s;
  if (!adam_prologue(a, r, h, bc1, bc2s)) {
    return;
  }

  Pack<T>* row[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    row[b] = reinterpret_cast<Pack<T>*>(a.x.data[b] + int64_t(r) * a.x.stride_r[b] + t0);
  }
  const int64_t packs_left = (a.g.T - t0) / kPack;

  Pack<T> v[NB][kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t i = int64_t(u) * kThreads + threadIdx.x;
    if (i < packs_left) {
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        v[b][u] = load_stream(row[b] + i);
      }
    }
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t i = int64_t(u) * kThreads + threadIdx.x;
    if (i < packs_left) {
#pragma unroll
      for (int k = 0; k < kPack; ++k) {
        opmath_t p = widen(v[0][u].v[k]);
        opmath_t m = widen(v[2][u].v[k]);
        opmath_t s = widen(v[3][u].v[k]);
        opmath_t mx = AMSGRAD ? widen(v[NB - 1][u].v[k]) : opmath_t(0);
        adam_element<opmath_t, ADAMW, AMSGRAD>(p, widen(v[1][u].v[k]), m, s, mx,
                                               h, a.maximize, bc1, bc2s);
        v[0][u].v[k] = narrow<T>(p);
        v[2][u].v[k] = narrow<T>(m);
        v[3][u].v[k] = narrow<T>(s);
        if constexpr (AMSGRAD) {
          v[NB - 1][u].v[k] = narrow<T>(mx);
        }
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if (b != 1) {
          store_stream(row[b] + i, v[b][u]);
        }
      }
    }
  }
}

template <typename T, bool ADAMW, bool AMSGRAD>
__global__ __launch_bounds__(kThreads) void adam_element_kernel(AdamArgs<T> a) {
  using opmath_t = op_t<T>;
  constexpr int NB = AMSGRAD ? 5 : 4;
  constexpr int kPer = kPack * kUnroll;
  uint32_t r;
  int64_t t0;
  tile_of_block(a.g, r, t0);
  AdamHyper h;
  opmath_t bc1, bc2s;
  if (!adam_prologue(a, r, h, bc1, bc2s)) {
    return;
  }

  T* base[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    base[b] = a.x.data[b] + int64_t(r) * a.x.stride_r[b];
  }
  T v[NB][kPer];
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int64_t t = t0 + int64_t(u) * kThreads + threadIdx.x;
    if (t < a.g.T) {
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        v[b][u] = base[b][t * a.x.stride_t[b]];
      }
    }
  }
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int64_t t = t0 + int64_t(u) * kThreads + threadIdx.x;
    if (t < a.g.T) {
      opmath_t p = widen(v[0][u]);
      opmath_t m = widen(v[2][u]);
      opmath_t s = widen(v[3][u]);
      opmath_t mx = AMSGRAD ? widen(v[NB - 1][u]) : opmath_t(0);
      adam_element<opmath_t, ADAMW, AMSGRAD>(p, widen(v[1][u]), m, s, mx, h,
                                             a.maximize, bc1, bc2s);
      base[0][t * a.x.stride_t[0]] = narrow<T>(p);
      base[2][t * a.x.stride_t[2]] = narrow<T>(m);
      base[3][t * a.x.stride_t[3]] = narrow<T>(s);
      if constexpr (AMSGRAD) {
        base[NB - 1][t * a.x.stride_t[NB - 1]] = narrow<T>(mx);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// SGD. The hyperparameters are carried as double inside the element math, as
// torch's ROCm `_fused_sgd_` takes them (checked on the MI355X: carrying them
// as float instead changes params and buffers by up to a few ulp).
// ---------------------------------------------------------------------------
using sgd_hyper_t = double;

template <typename T>
struct SgdArgs {
  Operands<T> x;  // param, grad, momentum_buffer
  const T* steps;
  const T* lr;
  const T* momentum;
  const T* dampening;
  const T* weight_decay;
  const uint8_t* mask;
  Grid g;
  bool maximize;
};

template <typename T>
__device__ __forceinline__ bool sgd_prologue(const SgdArgs<T>& a, uint32_t r,
                                             SgdHyper<sgd_hyper_t>& h,
                                             bool& is_first_step) {
  if (!a.mask[r]) {
    return false;
  }
  h.lr = static_cast<sgd_hyper_t>(widen(a.lr[r]));
  h.momentum = static_cast<sgd_hyper_t>(widen(a.momentum[r]));
  h.dampening = static_cast<sgd_hyper_t>(widen(a.dampening[r]));
  h.weight_decay = static_cast<sgd_hyper_t>(widen(a.weight_decay[r]));
  is_first_step = widen(a.steps[r]) == op_t<T>(1);
  return true;
}

template <typename T, bool HAS_BUF, bool NESTEROV>
__global__ __launch_bounds__(kThreads) void sgd_stream_kernel(SgdArgs<T> a) {
  using opmath_t = op_t<T>;
  constexpr int NB = HAS_BUF ? 3 : 2;
  uint32_t r;
  int64_t t0;
  tile_of_block(a.g, r, t0);
  SgdHyper<sgd_hyper_t> h;
  bool first;
  if (!sgd_prologue(a, r, h, first)) {
    return;
  }

  Pack<T>* row[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    row[b] = reinterpret_cast<Pack<T>*>(a.x.data[b] + int64_t(r) * a.x.stride_r[b] + t0);
  }
  const int64_t packs_left = (a.g.T - t0) / kPack;

  Pack<T> v[NB][kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t i = int64_t(u) * kThreads + threadIdx.x;
    if (i < packs_left) {
      v[0][u] = load_stream(row[0] + i);
      v[1][u] = load_stream(row[1] + i);
      // On a replica's first step the buffer is overwritten by the gradient
      // without being read, so it is not fetched.
      if (HAS_BUF && !first) {
        v[NB - 1][u] = load_stream(row[NB - 1] + i);
      }
    }
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t i = int64_t(u) * kThreads + threadIdx.x;
    if (i < packs_left) {
#pragma unroll
      for (int k = 0; k < kPack; ++k) {
        opmath_t p = widen(v[0][u].v[k]);
        opmath_t mb = (HAS_BUF && !first) ? widen(v[NB - 1][u].v[k]) : opmath_t(0);
        sgd_element<opmath_t, sgd_hyper_t, HAS_BUF, NESTEROV>(
            p, widen(v[1][u].v[k]), mb, h, a.maximize, first);
        v[0][u].v[k] = narrow<T>(p);
        if constexpr (HAS_BUF) {
          v[NB - 1][u].v[k] = narrow<T>(mb);
        }
      }
      store_stream(row[0] + i, v[0][u]);
      if constexpr (HAS_BUF) {
        store_stream(row[NB - 1] + i, v[NB - 1][u]);
      }
    }
  }
}

template <typename T, bool HAS_BUF, bool NESTEROV>
__global__ __launch_bounds__(kThreads) void sgd_element_kernel(SgdArgs<T> a) {
  using opmath_t = op_t<T>;
  constexpr int NB = HAS_BUF ? 3 : 2;
  constexpr int kPer = kPack * kUnroll;
  uint32_t r;
  int64_t t0;
  tile_of_block(a.g, r, t0);
  SgdHyper<sgd_hyper_t> h;
  bool first;
  if (!sgd_prologue(a, r, h, first)) {
    return;
  }

  T* base[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    base[b] = a.x.data[b] + int64_t(r) * a.x.stride_r[b];
  }
  T v[NB][kPer];
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int64_t t = t0 + int64_t(u) * kThreads + threadIdx.x;
    if (t < a.g.T) {
      v[0][u] = base[0][t * a.x.stride_t[0]];
      v[1][u] = base[1][t * a.x.stride_t[1]];
      if (HAS_BUF && !first) {
        v[NB - 1][u] = base[NB - 1][t * a.x.stride_t[NB - 1]];
      }
    }
  }
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int64_t t = t0 + int64_t(u) * kThreads + threadIdx.x;
    if (t < a.g.T) {
      opmath_t p = widen(v[0][u]);
      opmath_t mb = (HAS_BUF && !first) ? widen(v[NB - 1][u]) : opmath_t(0);
      sgd_element<opmath_t, sgd_hyper_t, HAS_BUF, NESTEROV>(
          p, widen(v[1][u]), mb, h, a.maximize, first);
      base[0][t * a.x.stride_t[0]] = narrow<T>(p);
      if constexpr (HAS_BUF) {
        base[NB - 1][t * a.x.stride_t[NB - 1]] = narrow<T>(mb);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Adagrad
// ---------------------------------------------------------------------------
template <typename T>
struct AdagradArgs {
  Operands<T> x;  // param, grad, state_sum
  const T* steps;
  const T* lr;
  const T* lr_decay;
  const T* weight_decay;
  const T* eps;
  const uint8_t* mask;
  Grid g;
  bool maximize;
};

template <typename T>
__device__ __forceinline__ bool adagrad_prologue(const AdagradArgs<T>& a,
                                                 uint32_t r, AdagradHyper& h) {
  if (!a.mask[r]) {
    return false;
  }
  const double lr = static_cast<double>(widen(a.lr[r]));
  const double lr_decay = static_cast<double>(widen(a.lr_decay[r]));
  h.weight_decay = static_cast<double>(widen(a.weight_decay[r]));
  h.eps = static_cast<double>(widen(a.eps[r]));
  h.corrected_lr = adagrad_corrected_lr(
      lr, lr_decay, static_cast<float>(widen(a.steps[r])));
  return true;
}

template <typename T>
__global__ __launch_bounds__(kThreads) void adagrad_stream_kernel(AdagradArgs<T> a) {
  using opmath_t = op_t<T>;
  constexpr int NB = 3;
  uint32_t r;
  int64_t t0;
  tile_of_block(a.g, r, t0);
  AdagradHyper h;
  if (!adagrad_prologue(a, r, h)) {
    return;
  }

  Pack<T>* row[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    row[b] = reinterpret_cast<Pack<T>*>(a.x.data[b] + int64_t(r) * a.x.stride_r[b] + t0);
  }
  const int64_t packs_left = (a.g.T - t0) / kPack;

  Pack<T> v[NB][kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t i = int64_t(u) * kThreads + threadIdx.x;
    if (i < packs_left) {
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        v[b][u] = load_stream(row[b] + i);
      }
    }
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t i = int64_t(u) * kThreads + threadIdx.x;
    if (i < packs_left) {
#pragma unroll
      for (int k = 0; k < kPack; ++k) {
        opmath_t p = widen(v[0][u].v[k]);
        opmath_t s = widen(v[2][u].v[k]);
        adagrad_element<opmath_t>(p, widen(v[1][u].v[k]), s, h, a.maximize);
        v[0][u].v[k] = narrow<T>(p);
        v[2][u].v[k] = narrow<T>(s);
      }
      store_stream(row[0] + i, v[0][u]);
      store_stream(row[2] + i, v[2][u]);
    }
  }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void adagrad_element_kernel(AdagradArgs<T> a) {
  using opmath_t = op_t<T>;
  constexpr int NB = 3;
  constexpr int kPer = kPack * kUnroll;
  uint32_t r;
  int64_t t0;
  tile_of_block(a.g, r, t0);
  AdagradHyper h;
  if (!adagrad_prologue(a, r, h)) {
    return;
  }

  T* base[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    base[b] = a.x.data[b] + int64_t(r) * a.x.stride_r[b];
  }
  T v[NB][kPer];
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int64_t t = t0 + int64_t(u) * kThreads + threadIdx.x;
    if (t < a.g.T) {
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        v[b][u] = base[b][t * a.x.stride_t[b]];
      }
    }
  }
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int64_t t = t0 + int64_t(u) * kThreads + threadIdx.x;
    if (t < a.g.T) {
      opmath_t p = widen(v[0][u]);
      opmath_t s = widen(v[2][u]);
      adagrad_element<opmath_t>(p, widen(v[1][u]), s, h, a.maximize);
      base[0][t * a.x.stride_t[0]] = narrow<T>(p);
      base[2][t * a.x.stride_t[2]] = narrow<T>(s);
    }
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
constexpr int kInvalid = static_cast<int>(hipErrorInvalidValue);

template <typename T>
bool fill_operands(const ts_rt_buf* bufs, int n, Operands<T>& x) {
  for (int b = 0; b < 5; ++b) {
    x.data[b] = nullptr;
    x.stride_r[b] = 0;
    x.stride_t[b] = 1;
  }
  for (int b = 0; b < n; ++b) {
    if (bufs[b].data == nullptr) {
      return false;
    }
    x.data[b] = static_cast<T*>(bufs[b].data);
    x.stride_r[b] = bufs[b].stride_r;
    x.stride_t[b] = bufs[b].stride_t;
  }
  return true;
}

// The 16-byte path needs every operand to have unit inner stride and every
// row start aligned to one pack, and T to be whole packs.
template <typename T>
bool streamable(const Operands<T>& x, int n, int64_t T_) {
  if (T_ % kPack != 0) {
    return false;
  }
  for (int b = 0; b < n; ++b) {
    if (x.stride_t[b] != 1 || x.stride_r[b] % kPack != 0 ||
        reinterpret_cast<uintptr_t>(x.data[b]) % (sizeof(T) * kPack) != 0) {
      return false;
    }
  }
  return true;
}

bool make_grid(int64_t R, int64_t T, Grid& g, uint32_t& blocks) {
  const int64_t tiles = (T + kTile - 1) / kTile;
  if (R <= 0 || T <= 0 || tiles > INT32_MAX || R > INT32_MAX / tiles) {
    return false;
  }
  g.T = T;
  g.tiles_per_row = static_cast<uint32_t>(tiles);
  blocks = static_cast<uint32_t>(R * tiles);
  return true;
}

template <typename T>
int launch_bump(void* steps, const uint8_t* mask, int64_t R, void* out_zero,
                hipStream_t stream) {
  const int64_t blocks = R > 0 ? (R + kThreads - 1) / kThreads : 1;
  if (blocks > INT32_MAX) {
    return kInvalid;
  }
  hipLaunchKernelGGL(bump_steps_kernel<T>, dim3(static_cast<uint32_t>(blocks)),
                     dim3(kThreads), 0, stream, static_cast<T*>(steps), mask, R,
                     static_cast<T*>(out_zero));
  return static_cast<int>(hipGetLastError());
}

// Runs the optional bump, then `launch` when there is any work.
// Empty tensors may carry null data pointers, so operands are only required
// where they are dereferenced: steps and mask when R > 0, the rest (checked
// inside `launch`) when there is at least one element.
template <typename T, typename Launch>
int run_step(void* steps, const uint8_t* mask, int64_t R, int64_t T_,
             uint32_t flags, void* out_zero, hipStream_t stream,
             Launch&& launch) {
  if (R < 0 || T_ < 0 || (R > 0 && (steps == nullptr || mask == nullptr))) {
    return kInvalid;
  }
  if ((flags & TS_BUMP_STEPS) != 0 || out_zero != nullptr) {
    if ((flags & TS_BUMP_STEPS) != 0 && R > 0) {
      const int err = launch_bump<T>(steps, mask, R, out_zero, stream);
      if (err != 0) {
        return err;
      }
    } else if (out_zero != nullptr) {
      const int err = launch_bump<T>(steps, mask, 0, out_zero, stream);
      if (err != 0) {
        return err;
      }
    }
  }
  if (R == 0 || T_ == 0) {
    return 0;
  }
  return launch();
}

template <typename T>
int adam_typed(const ts_rt_buf* bufs, void* steps, const void* lr,
               const void* beta1, const void* beta2, const void* eps,
               const void* wd, const uint8_t* mask, int64_t R, int64_t T_,
               uint32_t flags, void* out_zero, hipStream_t stream) {
  const bool amsgrad = (flags & TS_AMSGRAD) != 0;
  const bool adamw = (flags & TS_ADAMW) != 0;
  if (bufs == nullptr) {
    return kInvalid;
  }
  const bool work = R > 0 && T_ > 0;
  AdamArgs<T> a;
  if (work && (lr == nullptr || beta1 == nullptr || beta2 == nullptr || eps == nullptr ||
               wd == nullptr || !fill_operands<T>(bufs, amsgrad ? 5 : 4, a.x))) {
    return kInvalid;
  }
  a.steps = static_cast<const T*>(steps);
  a.lr = static_cast<const T*>(lr);
  a.beta1 = static_cast<const T*>(beta1);
  a.beta2 = static_cast<const T*>(beta2);
  a.eps = static_cast<const T*>(eps);
  a.weight_decay = static_cast<const T*>(wd);
  a.mask = mask;
  a.maximize = (flags & TS_MAXIMIZE) != 0;
  return run_step<T>(steps, mask, R, T_, flags, out_zero, stream, [&]() -> int {
    uint32_t blocks;
    if (!make_grid(R, T_, a.g, blocks)) {
      return kInvalid;
    }
    const bool stream_path = streamable(a.x, amsgrad ? 5 : 4, T_);
    const dim3 grid(blocks), block(kThreads);
#define CHURTEN_ADAM(W, A)                                                     \
  if (stream_path)                                                             \
    hipLaunchKernelGGL((adam_stream_kernel<T, W, A>), grid, block, 0, stream, a); \
  else                                                                         \
    hipLaunchKernelGGL((adam_element_kernel<T, W, A>), grid, block, 0, stream, a);
    if (adamw) {
      if (amsgrad) { CHURTEN_ADAM(true, true) } else { CHURTEN_ADAM(true, false) }
    } else {
      if (amsgrad) { CHURTEN_ADAM(false, true) } else { CHURTEN_ADAM(false, false) }
    }
#undef CHURTEN_ADAM
    return static_cast<int>(hipGetLastError());
  });
}

template <typename T>
int sgd_typed(const ts_rt_buf* bufs, void* steps, const void* lr,
              const void* momentum, const void* dampening, const void* wd,
              const uint8_t* mask, int64_t R, int64_t T_, uint32_t flags,
              void* out_zero, hipStream_t stream) {
  if (bufs == nullptr) {
    return kInvalid;
  }
  const bool work = R > 0 && T_ > 0;
  // bufs[2].data == NULL selects the buffer-less (depth-2) form.
  const bool has_buf = bufs[2].data != nullptr;
  const bool nesterov = (flags & TS_NESTEROV) != 0;
  if (work && nesterov && !has_buf) {
    return kInvalid;
  }
  SgdArgs<T> a;
  if (work && (lr == nullptr || momentum == nullptr || dampening == nullptr ||
               wd == nullptr || !fill_operands<T>(bufs, has_buf ? 3 : 2, a.x))) {
    return kInvalid;
  }
  a.steps = static_cast<const T*>(steps);
  a.lr = static_cast<const T*>(lr);
  a.momentum = static_cast<const T*>(momentum);
  a.dampening = static_cast<const T*>(dampening);
  a.weight_decay = static_cast<const T*>(wd);
  a.mask = mask;
  a.maximize = (flags & TS_MAXIMIZE) != 0;
  return run_step<T>(steps, mask, R, T_, flags, out_zero, stream, [&]() -> int {
    uint32_t blocks;
    if (!make_grid(R, T_, a.g, blocks)) {
      return kInvalid;
    }
    const bool stream_path = streamable(a.x, has_buf ? 3 : 2, T_);
    const dim3 grid(blocks), block(kThreads);
#define CHURTEN_SGD(B, N)                                                      \
  if (stream_path)                                                             \
    hipLaunchKernelGGL((sgd_stream_kernel<T, B, N>), grid, block, 0, stream, a); \
  else                                                                         \
    hipLaunchKernelGGL((sgd_element_kernel<T, B, N>), grid, block, 0, stream, a);
    if (has_buf) {
      if (nesterov) { CHURTEN_SGD(true, true) } else { CHURTEN_SGD(true, false) }
    } else {
      CHURTEN_SGD(false, false)
    }
#undef CHURTEN_SGD
    return static_cast<int>(hipGetLastError());
  });
}

template <typename T>
int adagrad_typed(const ts_rt_buf* bufs, void* steps, const void* lr,
                  const void* lr_decay, const void* wd, const void* eps,
                  const uint8_t* mask, int64_t R, int64_t T_, uint32_t flags,
                  void* out_zero, hipStream_t stream) {
  if (bufs == nullptr) {
    return kInvalid;
  }
  const bool work = R > 0 && T_ > 0;
  AdagradArgs<T> a;
  if (work && (lr == nullptr || lr_decay == nullptr || wd == nullptr || eps == nullptr ||
               !fill_operands<T>(bufs, 3, a.x))) {
    return kInvalid;
  }
  a.steps = static_cast<const T*>(steps);
  a.lr = static_cast<const T*>(lr);
  a.lr_decay = static_cast<const T*>(lr_decay);
  a.weight_decay = static_cast<const T*>(wd);
  a.eps = static_cast<const T*>(eps);
  a.mask = mask;
  a.maximize = (flags & TS_MAXIMIZE) != 0;
  return run_step<T>(steps, mask, R, T_, flags, out_zero, stream, [&]() -> int {
    uint32_t blocks;
    if (!make_grid(R, T_, a.g, blocks)) {
      return kInvalid;
    }
    const dim3 grid(blocks), block(kThreads);
    if (streamable(a.x, 3, T_)) {
      hipLaunchKernelGGL(adagrad_stream_kernel<T>, grid, block, 0, stream, a);
    } else {
      hipLaunchKernelGGL(adagrad_element_kernel<T>, grid, block, 0, stream, a);
    }
    return static_cast<int>(hipGetLastError());
  });
}

}  // namespace
}  // namespace churten

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" {

int ts_version(void) { return 100; }

int ts_bump_steps(ts_dtype dtype, void* state_steps, const uint8_t* active_mask,
                  int64_t R, void* out_zero, void* stream) {
  using namespace churten;
  if (R < 0 || (R > 0 && (state_steps == nullptr || active_mask == nullptr))) {
    return kInvalid;
  }
  auto s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case TS_FLOAT32: return launch_bump<float>(state_steps, active_mask, R, out_zero, s);
    case TS_FLOAT64: return launch_bump<double>(state_steps, active_mask, R, out_zero, s);
    case TS_FLOAT16: return launch_bump<_Float16>(state_steps, active_mask, R, out_zero, s);
    case TS_BFLOAT16: return launch_bump<bf16_t>(state_steps, active_mask, R, out_zero, s);
  }
  return kInvalid;
}

int ts_adam_step(const ts_rt_buf* bufs, ts_dtype dtype, void* state_steps,
                 const void* lr, const void* beta1, const void* beta2,
                 const void* eps, const void* weight_decay,
                 const uint8_t* active_mask, int64_t R, int64_t T,
                 uint32_t flags, void* out_zero, void* stream) {
  using namespace churten;
  auto s = static_cast<hipStream_t>(stream);
#define CHURTEN_CALL(TY) \
  adam_typed<TY>(bufs, state_steps, lr, beta1, beta2, eps, weight_decay, active_mask, R, T, flags, out_zero, s)
  switch (dtype) {
    case TS_FLOAT32: return CHURTEN_CALL(float);
    case TS_FLOAT64: return CHURTEN_CALL(double);
    case TS_FLOAT16: return CHURTEN_CALL(_Float16);
    case TS_BFLOAT16: return CHURTEN_CALL(bf16_t);
  }
#undef CHURTEN_CALL
  return kInvalid;
}

int ts_sgd_step(const ts_rt_buf* bufs, ts_dtype dtype, void* state_steps,
                const void* lr, const void* momentum, const void* dampening,
                const void* weight_decay, const uint8_t* active_mask,
                int64_t R, int64_t T, uint32_t flags, void* out_zero,
                void* stream) {
  using namespace churten;
  auto s = static_cast<hipStream_t>(stream);
#define CHURTEN_CALL(TY) \
  sgd_typed<TY>(bufs, state_steps, lr, momentum, dampening, weight_decay, active_mask, R, T, flags, out_zero, s)
  switch (dtype) {
    case TS_FLOAT32: return CHURTEN_CALL(float);
    case TS_FLOAT64: return CHURTEN_CALL(double);
    case TS_FLOAT16: return CHURTEN_CALL(_Float16);
    case TS_BFLOAT16: return CHURTEN_CALL(bf16_t);
  }
#undef CHURTEN_CALL
  return kInvalid;
}

int ts_adagrad_step(const ts_rt_buf* bufs, ts_dtype dtype, void* state_steps,
                    const void* lr, const void* lr_decay,
                    const void* weight_decay, const void* eps,
                    const uint8_t* active_mask, int64_t R, int64_t T,
                    uint32_t flags, void* out_zero, void* stream) {
  using namespace churten;
  auto s = static_cast<hipStream_t>(stream);
#define CHURTEN_CALL(TY) \
  adagrad_typed<TY>(bufs, state_steps, lr, lr_decay, weight_decay, eps, active_mask, R, T, flags, out_zero, s)
  switch (dtype) {
    case TS_FLOAT32: return CHURTEN_CALL(float);
    case TS_FLOAT64: return CHURTEN_CALL(double);
    case TS_FLOAT16: return CHURTEN_CALL(_Float16);
    case TS_BFLOAT16: return CHURTEN_CALL(bf16_t);
  }
#undef CHURTEN_CALL
  return kInvalid;
}

}  // extern "C"
