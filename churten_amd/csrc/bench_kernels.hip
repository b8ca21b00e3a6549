// bench_kernels.hip -- measurement and test aids, not part of the C ABI in
// include/. cb_traffic: the Adam step's HBM access pattern without its
// arithmetic, so bench.py can set the update kernel's rate against what the
// same traffic reaches on the same buffers in the same process.
// cb_narrow_bf16 / cb_narrow_f16: the kernels' float -> bfloat16 / half
// narrowing over an array, for the tests that check them against torch's
// conversions on every float bit pattern (cb_narrow2_bf16: the paired form the
// drivers store packs with). cb_sqrt_rn: the update's float square root over
// an array, for the test that checks it against torch's. cb_div_bc2s: Adam's sqrt(v) /
// bias_correction2_sqrt as the float update computes it (a multiply by the
// divisor's double reciprocal), for the tests that check it against a true
// division. cb_div_tiles: the streaming driver's division of a workgroup
// index by the tiles per row, for the test that checks it against integer
// division.
//
// Same decomposition as the streaming driver at float32: one-wave workgroups,
// tiles of (replica, tile) pairs, frozen replicas skipped, one or two
// non-temporal 16-byte packs per thread per operand (256- or 512-element
// tiles). Modes:
//   0  read params, grads, exp_avg, exp_avg_sq; write params, exp_avg,
//      exp_avg_sq (28 B per active element, the Adam step's traffic)
//   1  the four reads only (16 B)
//   2  the three writes only (12 B; the written values are `c`)
//   3  mode 0 with bfloat16 moments next to float32 params and grads, as
//      Adam with TS_STATE_BF16 moves them: `m` and `v` point at (R, T)
//      bfloat16 buffers, read and written 8 bytes (4 values) per thread per
//      pack, params and grads 16 bytes (20 B per active element)
// Mode 0 writes x + g * c, so with c = 0 it leaves finite values unchanged;
// mode 3 writes params likewise and flips the lowest bit of every moment
// value when c != 0.

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "optim_drivers.h"
#include "optim_math.h"

namespace {

constexpr int kThreads = 64;

using F4 = float __attribute__((ext_vector_type(4)));

__device__ __forceinline__ F4 ld(const F4* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void st(F4* p, F4 v) { __builtin_nontemporal_store(v, p); }

template <int MODE, int kUnroll>
__global__ __launch_bounds__(kThreads) void traffic_kernel(float* p, const float* g, float* m,
                                                           float* v, const uint8_t* mask,
                                                           int64_t T, uint32_t tiles, float c,
                                                           float* sink) {
  constexpr int64_t kTile = int64_t(kThreads) * 4 * kUnroll;
  const uint32_t b = blockIdx.x;
  const uint32_t r = b / tiles;
  const int64_t t0 = int64_t(b - r * tiles) * kTile;
  if (!mask[r]) return;
  const int64_t base = int64_t(r) * T + t0;
  F4* const P = reinterpret_cast<F4*>(p + base);
  const F4* const G = reinterpret_cast<const F4*>(g + base);
  F4* const M = reinterpret_cast<F4*>(m + base);
  F4* const V = reinterpret_cast<F4*>(v + base);
  const int64_t left = (T - t0) / 4;
  F4 a[kUnroll], bb[kUnroll], cc[kUnroll], d[kUnroll];
  if constexpr (MODE != 2) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = int64_t(u) * kThreads + threadIdx.x;
      if (i < left) {
        a[u] = ld(P + i);
        bb[u] = ld(G + i);
        cc[u] = ld(M + i);
        d[u] = ld(V + i);
      }
    }
  }
  F4 acc = F4(0.0f);
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t i = int64_t(u) * kThreads + threadIdx.x;
    if (i < left) {
      if constexpr (MODE == 0) {
        st(P + i, a[u] + bb[u] * c);
        st(M + i, cc[u] + bb[u] * c);
        st(V + i, d[u] + bb[u] * c);
      } else if constexpr (MODE == 1) {
        acc += a[u] + bb[u] + cc[u] + d[u];
      } else {
        const F4 k = F4(c);
        st(P + i, k);
        st(M + i, k);
        st(V + i, k);
      }
    }
  }
  if constexpr (MODE == 1) {
    // keeps the reads: the host passes a `c` no sum of the data reaches
    if (acc.x + acc.y + acc.z + acc.w == c) sink[0] = acc.x;
  }
}

using U2 = uint32_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ U2 ld(const U2* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void st(U2* p, U2 v) { __builtin_nontemporal_store(v, p); }

// Mode 3 of cb_traffic: tiles as traffic_kernel's, moments as 4-value
// bfloat16 packs.
template <int kUnroll>
__global__ __launch_bounds__(kThreads) void traffic_bf16_kernel(float* p, const float* g,
                                                                uint16_t* m, uint16_t* v,
                                                                const uint8_t* mask, int64_t T,
                                                                uint32_t tiles, float c) {
  constexpr int64_t kTile = int64_t(kThreads) * 4 * kUnroll;
  const uint32_t b = blockIdx.x;
  const uint32_t r = b / tiles;
  const int64_t t0 = int64_t(b - r * tiles) * kTile;
  if (!mask[r]) return;
  const int64_t base = int64_t(r) * T + t0;
  F4* const P = reinterpret_cast<F4*>(p + base);
  const F4* const G = reinterpret_cast<const F4*>(g + base);
  U2* const M = reinterpret_cast<U2*>(m + base);
  U2* const V = reinterpret_cast<U2*>(v + base);
  const int64_t left = (T - t0) / 4;
  const uint32_t flip = c != 0.0f ? 0x00010001u : 0u;  // the lowest bit of both values
  F4 a[kUnroll], bb[kUnroll];
  U2 cc[kUnroll], d[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t i = int64_t(u) * kThreads + threadIdx.x;
    if (i < left) {
      a[u] = ld(P + i);
      bb[u] = ld(G + i);
      cc[u] = ld(M + i);
      d[u] = ld(V + i);
    }
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t i = int64_t(u) * kThreads + threadIdx.x;
    if (i < left) {
      st(P + i, a[u] + bb[u] * c);
      st(M + i, cc[u] ^ flip);
      st(V + i, d[u] ^ flip);
    }
  }
}

__global__ __launch_bounds__(256) void narrow_bf16_kernel(const float* in, uint16_t* out,
                                                          int64_t n) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) out[i] = churten::narrow<churten::bf16_t>(in[i]).bits;
}

__global__ __launch_bounds__(256) void narrow2_bf16_kernel(const float* in, uint32_t* out,
                                                           int64_t pairs) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i < pairs) out[i] = churten::narrow2_bf16(in[2 * i], in[2 * i + 1]);
}

template <bool ZEROS>
__global__ __launch_bounds__(256) void sqrt_rn_kernel(const float* in, float* out, int64_t n) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) out[i] = churten::sqrt_rn<ZEROS>(in[i]);
}

// b_stride 0: one divisor for every element; 1: one per element.
__global__ __launch_bounds__(256) void div_bc2s_kernel(const float* x, const float* b,
                                                       int64_t b_stride, float* out, int64_t n) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) {
    const churten::AdamConsts<float> c = churten::adam_consts<float>(1.0, 1.0f, b[i * b_stride]);
    out[i] = churten::adam_div_bc2s(x[i], c.bc2s_div);
  }
}

__global__ __launch_bounds__(256) void div_tiles_kernel(churten::Grid g, const uint32_t* m,
                                                        uint32_t* q, int64_t n) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) q[i] = churten::div_tiles(g, m[i]);
}

__global__ __launch_bounds__(256) void narrow_f16_kernel(const float* in, uint16_t* out,
                                                         int64_t n) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) out[i] = __builtin_bit_cast(uint16_t, churten::narrow<_Float16>(in[i]));
}

}  // namespace

// q[i] = m[i] / d as the streaming driver divides a workgroup index by the
// tiles per row (the constants from set_div_tiles, the quotient from
// div_tiles). Returns 0, 1 on bad arguments, or the HIP error code.
extern "C" int cb_div_tiles(uint32_t d, const uint32_t* m, uint32_t* q, int64_t n,
                            hipStream_t stream) {
  if (d == 0 || n <= 0 || n > int64_t(UINT32_MAX) * 256) return 1;
  churten::Grid g{};
  g.tiles_per_row = d;
  churten::set_div_tiles(g);
  const uint32_t blocks = static_cast<uint32_t>((n + 255) / 256);
  hipLaunchKernelGGL(div_tiles_kernel, dim3(blocks), dim3(256), 0, stream, g, m, q, n);
  return static_cast<int>(hipGetLastError());
}

// out[i] = the half bits the update kernels store for the float in[i].
extern "C" int cb_narrow_f16(const float* in, uint16_t* out, int64_t n, hipStream_t stream) {
  if (n <= 0 || n > int64_t(UINT32_MAX) * 256) return 1;
  const uint32_t blocks = static_cast<uint32_t>((n + 255) / 256);
  hipLaunchKernelGGL(narrow_f16_kernel, dim3(blocks), dim3(256), 0, stream, in, out, n);
  return static_cast<int>(hipGetLastError());
}

// out[i] = the bfloat16 bits the update kernels store for the float in[i].
// Returns 0, 1 on bad arguments, or the HIP error code.
extern "C" int cb_narrow_bf16(const float* in, uint16_t* out, int64_t n, hipStream_t stream) {
  if (n <= 0 || n > int64_t(UINT32_MAX) * 256) return 1;
  const uint32_t blocks = static_cast<uint32_t>((n + 255) / 256);
  hipLaunchKernelGGL(narrow_bf16_kernel, dim3(blocks), dim3(256), 0, stream, in, out, n);
  return static_cast<int>(hipGetLastError());
}

// out[i] = the two bfloat16 (low half first) the drivers store for the floats
// in[2i], in[2i + 1]. Returns 0, 1 on bad arguments, or the HIP error code.
extern "C" int cb_narrow2_bf16(const float* in, uint32_t* out, int64_t pairs,
                               hipStream_t stream) {
  if (pairs <= 0 || pairs > int64_t(UINT32_MAX) * 256) return 1;
  const uint32_t blocks = static_cast<uint32_t>((pairs + 255) / 256);
  hipLaunchKernelGGL(narrow2_bf16_kernel, dim3(blocks), dim3(256), 0, stream, in, out, pairs);
  return static_cast<int>(hipGetLastError());
}

// out[i] = the float square root the update kernels take of in[i]; zeros != 0:
// the form of the float16-state policies (zero-only wavefronts on the short
// path).
extern "C" int cb_sqrt_rn(const float* in, float* out, int64_t n, int zeros,
                          hipStream_t stream) {
  if (n <= 0 || n > int64_t(UINT32_MAX) * 256) return 1;
  const uint32_t blocks = static_cast<uint32_t>((n + 255) / 256);
  if (zeros) {
    hipLaunchKernelGGL(sqrt_rn_kernel<true>, dim3(blocks), dim3(256), 0, stream, in, out, n);
  } else {
    hipLaunchKernelGGL(sqrt_rn_kernel<false>, dim3(blocks), dim3(256), 0, stream, in, out, n);
  }
  return static_cast<int>(hipGetLastError());
}

// out[i] = x[i] / b[i * b_stride] as the float Adam update divides sqrt(v) by
// bias_correction2_sqrt (b_stride 0 or 1). Returns 0, 1 on bad arguments, or
// the HIP error code.
extern "C" int cb_div_bc2s(const float* x, const float* b, int64_t b_stride, float* out,
                           int64_t n, hipStream_t stream) {
  if (n <= 0 || n > int64_t(UINT32_MAX) * 256 || (b_stride != 0 && b_stride != 1)) return 1;
  const uint32_t blocks = static_cast<uint32_t>((n + 255) / 256);
  hipLaunchKernelGGL(div_bc2s_kernel, dim3(blocks), dim3(256), 0, stream, x, b, b_stride, out,
                     n);
  return static_cast<int>(hipGetLastError());
}

// The pattern over the active rows of four row-major (R, T) buffers (float32;
// in mode 3 `m` and `v` hold bfloat16): T a multiple of 4, every base 16-byte
// aligned, `mask` R bytes, `packs` 1 or 2 per thread. `lds` is the dynamic LDS
// per workgroup (a residency cap, as the streaming driver's). Returns 0, 1 on
// bad arguments, or the HIP error code.
extern "C" int cb_traffic(int mode, float* p, const float* g, float* m, float* v,
                          const uint8_t* mask, int64_t R, int64_t T, float c, uint32_t lds,
                          int packs, float* sink, hipStream_t stream) {
  if (R <= 0 || T <= 0 || T % 4 != 0 || mode < 0 || mode > 3 || packs < 1 || packs > 2) return 1;
  for (const void* q : {static_cast<const void*>(p), static_cast<const void*>(g),
                        static_cast<const void*>(m), static_cast<const void*>(v)}) {
    if (reinterpret_cast<uintptr_t>(q) % 16 != 0) return 1;
  }
  const int64_t tile = int64_t(kThreads) * 4 * packs;
  const int64_t tiles = (T + tile - 1) / tile;
  if (tiles > INT32_MAX || R > INT32_MAX / tiles) return 1;
  const dim3 grid(static_cast<uint32_t>(R * tiles)), block(kThreads);
  const uint32_t t32 = static_cast<uint32_t>(tiles);
  if (mode == 3) {
    uint16_t* const mb = reinterpret_cast<uint16_t*>(m);
    uint16_t* const vb = reinterpret_cast<uint16_t*>(v);
    if (packs == 1) {
      hipLaunchKernelGGL(traffic_bf16_kernel<1>, grid, block, lds, stream, p, g, mb, vb, mask,
                         T, t32, c);
    } else {
      hipLaunchKernelGGL(traffic_bf16_kernel<2>, grid, block, lds, stream, p, g, mb, vb, mask,
                         T, t32, c);
    }
    return static_cast<int>(hipGetLastError());
  }
  using K = void (*)(float*, const float*, float*, float*, const uint8_t*, int64_t, uint32_t,
                     float, float*);
  const K kernels[3][2] = {{traffic_kernel<0, 1>, traffic_kernel<0, 2>},
                           {traffic_kernel<1, 1>, traffic_kernel<1, 2>},
                           {traffic_kernel<2, 1>, traffic_kernel<2, 2>}};
  hipLaunchKernelGGL(kernels[mode][packs - 1], grid, block, lds, stream, p, g, m, v, mask, T, t32,
                     c, sink);
  return static_cast<int>(hipGetLastError());
}
