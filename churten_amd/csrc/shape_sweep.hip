// shape_sweep.hip -- measurement aid, not part of the library: times the
// production update kernels with their launch shape overridden, on buffers the
// size of a BASELINE config (default config 5: 128 replicas x 25,171,968
// elements, ~90% of the replicas active; config 2: 100 x 265,484, ~75%;
// config 4: 64 x 545,100, all), through the production launch path
// (launch_dense / launch_segments with a workspace). This is what the shape
// constants of the policies in optim_drivers.h were chosen from.
//
// Streaming families vary packs per thread (1, 2, 4) and the residency cap
// (none, 3-20 one-wave workgroups per CU); the segmented family varies
// threads per workgroup (64, 128), packs (1, 2) and the cap, next to the dense
// update on the same state. Every variant is timed in each of several
// interleaved rounds (2 untimed launches, then 15 timed between two events);
// the summary gives the best and mean rate over the rounds, in GB/s of the
// active rows' algorithmic bytes.
//
// Build and run (one family per process; SWEEP_FAMILY limits the build to it):
//   hipcc --offload-arch=gfx950 -O3 -std=c++17 \
//     -Xclang -target-feature -Xclang -packed-fp32-ops \
//     -DSWEEP_FAMILY=adam_bf16state churten_amd/csrc/shape_sweep.hip -o shape_sweep
//   ./shape_sweep adam_bf16state [cfg2|cfg4|cfg5|RxTxPCT]
// Families: adam_f32 adam_ams_f32 adam_bf16state adam_f16 adam_bf16 sgd_f32
// sgd_bf16state sgd_f16 sgd_bf16 adagrad_f32 adagrad_bf16state adagrad_f16
// adagrad_bf16 seg_adam_f32 (config 5 only); the math families math_adam_f32
// math_adam_bf16state math_adam_f16 math_adam_bf16 math_adagrad_f32
// math_adagrad_f16 math_adagrad_bf16 time the shipped shape with the element
// math's square root as std::sqrt and as the shipped sqrt_rn (bit-identical). Config 5 needs about 65 GB of
// device memory.

#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <functional>
#include <string>
#include <utility>
#include <vector>

#include "optim_drivers.h"

using namespace churten;

namespace {

#define SWEEP_CHECK(x)                                                              \
  do {                                                                              \
    const hipError_t e_ = (x);                                                      \
    if (e_ != hipSuccess) {                                                         \
      fprintf(stderr, "%s:%d: %s\n", __FILE__, __LINE__, hipGetErrorString(e_));   \
      exit(1);                                                                      \
    }                                                                               \
  } while (0)

// A policy with its streaming shape replaced (with and without a workspace,
// and for launches that fit the MALL, which run uncapped whatever CAP says).
template <typename Base, int U, int CAP, int NTH = 64>
struct StreamShape : Base {
  static constexpr int kStreamBlock = NTH;
  static constexpr int kStreamBlockSmall = NTH;
  static constexpr int kStreamUnrollPre = U;
  static constexpr int kStreamUnroll = U;
  static constexpr int kStreamUnrollSmall = U;
  static constexpr uint32_t kStreamLdsPre = CAP ? lds_for_residency(CAP) : 0u;
  static constexpr uint32_t kStreamLds = kStreamLdsPre;
  static constexpr uint32_t kStreamLdsMid = kStreamLdsPre;
};

// A policy with its segmented shape (with a workspace) replaced; the cap is
// passed at launch.
template <typename Base, int NTH, int U>
struct SegmentShape : Base {
  static constexpr int kSegmentThreadsPre = NTH;
  static constexpr int kSegmentUnrollPre = U;
};

// The same policy with hipcc's std::sqrt in its element math instead of
// sqrt_rn (bit-identical), for the math family. Adam without AdamW, and
// Adagrad with fp64 math.
template <typename Base>
struct PerElementStdSqrt : Base {
  using M = typename Base::M;
  // every pack through update() below (not float16 Adagrad's pair form)
  static constexpr bool kVariant = false;
  __device__ static void update(M& p, M g, M (&s)[Base::NS], const typename Base::Rep& rep,
                                bool maximize) {
    if constexpr (Base::NS >= 2) {  // Adam
      M mx = M(0);
      if constexpr (Base::NS == 3) mx = s[2];
      const M v = adam_moments<M, false, Base::NS == 3>(p, g, s[0], s[1], mx, rep.h, maximize);
      adam_finish(p, s[0], std::sqrt(v), rep.h, rep.c);
      if constexpr (Base::NS == 3) s[2] = mx;
    } else {  // Adagrad (fp64 math)
      adagrad_sum<M>(p, g, s[0], rep.h, maximize);
      adagrad_finish<M>(p, g, std::sqrt(s[0]), rep.h);
    }
  }
};

// Deterministic pseudo-random fill: x in (-scale/2, scale/2), or positive.
template <typename T>
__global__ void fill_kernel(T* x, int64_t n, uint32_t seed, float scale, bool positive) {
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += int64_t(gridDim.x) * 256) {
    uint32_t h = static_cast<uint32_t>(i) * 2654435761u ^ seed;
    h ^= h >> 15;
    h *= 2246822519u;
    h ^= h >> 13;
    float u = static_cast<float>(h & 0xFFFFFF) / 16777216.0f - 0.5f;
    if (positive) u = fabsf(u) + 1e-3f;
    x[i] = narrow<T>(op_t<T>(u * scale));
  }
}

template <typename T>
T host_value(double d) {
  return static_cast<T>(d);
}
template <>
bf16_t host_value<bf16_t>(double d) {  // round to nearest even
  const float f = static_cast<float>(d);
  uint32_t u;
  memcpy(&u, &f, 4);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return bf16_t{static_cast<uint16_t>(u >> 16)};
}

// The workload: replicas, elements per replica, percent of replicas active.
struct Workload {
  int64_t R, T;
  int active_pct;
};
Workload g_work{128, 25171968, 90};

// The (R, T) operands (params, grads, NS state buffers), the (R,) vectors, a
// mask with the workload's share of active replicas and the workspace.
template <typename T, typename S, int NS>
struct State {
  const int64_t R = g_work.R, T_ = g_work.T;
  void* buf[5] = {};
  T* steps = nullptr;
  T* h[5] = {};
  uint8_t* mask = nullptr;
  double* ws = nullptr;
  int active = 0;

  State() {
    const int64_t n = R * T_;
    for (int b = 0; b < 2 + NS; ++b) {
      const size_t es = b < 2 ? sizeof(T) : sizeof(S);
      SWEEP_CHECK(hipMalloc(&buf[b], n * es));
      if (b < 2) {
        hipLaunchKernelGGL(fill_kernel<T>, dim3(4096), dim3(256), 0, 0, static_cast<T*>(buf[b]),
                           n, 17u * b + 1, b == 0 ? 0.04f : 2e-3f, false);
      } else {
        hipLaunchKernelGGL(fill_kernel<S>, dim3(4096), dim3(256), 0, 0, static_cast<S*>(buf[b]),
                           n, 17u * b + 1, b == 2 ? 2e-3f : 1e-4f, b > 2);
      }
    }
    std::vector<uint8_t> hm(R);
    uint32_t s = 1005;
    for (auto& x : hm) {
      s = s * 1664525u + 1013904223u;
      x = static_cast<int>((s >> 8) % 100) < g_work.active_pct;
      active += x;
    }
    SWEEP_CHECK(hipMalloc(&mask, R));
    SWEEP_CHECK(hipMemcpy(mask, hm.data(), R, hipMemcpyHostToDevice));
    std::vector<T> hv(R);
    const auto upload = [&](T*& d, const std::function<double(int)>& f) {
      for (int i = 0; i < R; ++i) hv[i] = host_value<T>(f(i));
      SWEEP_CHECK(hipMalloc(&d, R * sizeof(T)));
      SWEEP_CHECK(hipMemcpy(d, hv.data(), R * sizeof(T), hipMemcpyHostToDevice));
    };
    // step in [1, 10000]; hypers valid for every optimizer's reading of them
    upload(steps, [](int i) { return 1 + (i * 7919) % 10000; });
    upload(h[0], [](int i) { return 1e-4 * (1 + i % 7); });
    upload(h[1], [](int) { return 0.9; });
    upload(h[2], [](int) { return 0.999; });
    upload(h[3], [](int) { return 1e-8; });
    upload(h[4], [](int) { return 0.0; });
    SWEEP_CHECK(hipMalloc(&ws, R * kPreStride * sizeof(double)));
    SWEEP_CHECK(hipDeviceSynchronize());
  }

  Call call(ts_rt_buf* bufs, int nh, bool with_grad = true) {
    for (int b = 0; b < 5; ++b) {
      bufs[b].data = buf[b];
      bufs[b].stride_r = T_;
      bufs[b].stride_t = 1;
    }
    if (!with_grad) bufs[1].data = nullptr;
    Call c = make_call(bufs, steps, {h[0], h[1], h[2], h[3], h[4]}, mask, R, T_, 0, nullptr,
                       nullptr, ws, R * kPreStride * sizeof(double));
    c.nh = nh;
    return c;
  }
};

struct Variant {
  std::string name;
  std::function<int()> launch;
  std::vector<float> ms;
};

void time_variants(std::vector<Variant>& v, double bytes, int rounds) {
  hipEvent_t a, b;
  SWEEP_CHECK(hipEventCreate(&a));
  SWEEP_CHECK(hipEventCreate(&b));
  for (int round = 0; round < rounds; ++round) {
    for (auto& x : v) {
      for (int w = 0; w < 2; ++w) SWEEP_CHECK(static_cast<hipError_t>(x.launch()));
      constexpr int kTimed = 15;
      SWEEP_CHECK(hipEventRecord(a));
      for (int w = 0; w < kTimed; ++w) x.launch();
      SWEEP_CHECK(hipEventRecord(b));
      SWEEP_CHECK(hipEventSynchronize(b));
      float ms = 0;
      SWEEP_CHECK(hipEventElapsedTime(&ms, a, b));
      x.ms.push_back(ms / kTimed);
      printf("round %d %-24s %.3f ms\n", round, x.name.c_str(), ms / kTimed);
      fflush(stdout);
    }
  }
  printf("== summary: %d rounds, GB/s of %.4g algorithmic bytes per launch\n", rounds, bytes);
  for (auto& x : v) {
    const float best = *std::min_element(x.ms.begin(), x.ms.end());
    float sum = 0;
    for (float t : x.ms) sum += t;
    printf("%-24s best %.3f ms %7.1f GB/s  mean %7.1f GB/s\n", x.name.c_str(), best,
           bytes / (best * 1e-3) / 1e9, bytes / (sum / x.ms.size() * 1e-3) / 1e9);
  }
}

template <typename P, typename St>
int dense(St& st, int nh) {
  ts_rt_buf bufs[5];
  return launch_dense<P>(st.call(bufs, nh), 2 + P::NS);
}

template <typename Base, typename St, int U, int... CAPS>
void add_stream(std::vector<Variant>& v, St& st, int nh, std::integer_sequence<int, CAPS...>) {
  (v.push_back({"packs=" + std::to_string(U) + " cap=" + std::to_string(CAPS),
                [&st, nh] { return dense<StreamShape<Base, U, CAPS>>(st, nh); },
                {}}),
   ...);
}

// Streaming family: policy Base over State<T, S, NS>; nh hyperparameter vectors;
// bytes per active element.
template <typename Base, int NS>
void stream_family(int nh, int bytes_per_elem) {
  State<typename Base::T, typename Base::S, NS> st;
  std::vector<Variant> v;
  using caps = std::integer_sequence<int, 0, 3, 4, 6, 8, 10, 12, 14, 16, 20>;
  add_stream<Base, decltype(st), 1>(v, st, nh, caps{});
  add_stream<Base, decltype(st), 2>(v, st, nh, caps{});
  add_stream<Base, decltype(st), 4>(v, st, nh, caps{});
  time_variants(v, double(st.active) * st.T_ * bytes_per_elem, 3);
}

// Math family: the policy at its shipped shape with std::sqrt and with
// sqrt_rn, interleaved in one process (so on the same buffers and pages), 5
// rounds.
template <typename Base, int NS>
void math_family(int nh, int bytes_per_elem) {
  State<typename Base::T, typename Base::S, NS> st;
  std::vector<Variant> v;
  v.push_back({"std::sqrt", [&st, nh] { return dense<PerElementStdSqrt<Base>>(st, nh); }, {}});
  v.push_back({"sqrt_rn (shipped)", [&st, nh] { return dense<Base>(st, nh); }, {}});
  time_variants(v, double(st.active) * st.T_ * bytes_per_elem, 5);
}

// The segmented float32 Adam update: the gradient as config 5's twelve
// per-parameter (R, numel) tensors, the consolidated gradient not written.
template <typename P, typename St>
int segmented(St& st, const std::vector<ts_segment>& segs, uint32_t cap) {
  ts_rt_buf bufs[5];
  const Call c = st.call(bufs, 5, false);
  // launch_segments with the residency reservation `cap` (the production
  // launch runs uncapped): the same walk, launched here directly
  using T = typename P::T;
  SegArgs<P> a;
  if (!fill_kargs<P>(c, 4, a.k, true)) return 1;
  a.k.g = Grid{c.T, 0, 0, 0};
  const bool vec_rows = rows_streamable<P>(a.k.x, 4, a.k.g.res0, a.k.g.rmod);
  const SegmentWalk walk{segs.data(), static_cast<int>(segs.size()), c.T, true};
  const int err = launch_prep<P>(c, a.k.vec);
  if (err != 0) return err;
  return launch_walk<T>(walk, c.R, segment_tile<P, true>(), vec_rows, a, a.seg,
                        segment_kernel<P, false, true>, c.stream,
                        cap ? lds_for_residency(cap) : 0u, segment_threads<P, true>());
}

template <typename Base, typename St, int NTH, int U>
void add_segment(std::vector<Variant>& v, St& st, const std::vector<ts_segment>& segs) {
  for (uint32_t cap : {0u, 8u, 12u, 14u, 20u}) {
    v.push_back({"threads=" + std::to_string(NTH) + " packs=" + std::to_string(U) +
                     " cap=" + std::to_string(cap),
                 [&st, &segs, cap] {
                   return segmented<SegmentShape<Base, NTH, U>>(st, segs, cap);
                 },
                 {}});
  }
}

void segment_family() {
  using Base = AdamPolicy<float, false, false>;
  State<float, float, 2> st;
  const int64_t sizes[12] = {4096 * 1024, 4096 * 1024, 4096 * 1024, 4096 * 1024,
                             1024 * 4096, 1024 * 4096, 1024, 1024, 1024, 1024, 1024, 1024};
  std::vector<ts_segment> segs;
  int64_t col = 0;
  for (int i = 0; i < 12; ++i) {
    void* d = nullptr;
    SWEEP_CHECK(hipMalloc(&d, st.R * sizes[i] * sizeof(float)));
    hipLaunchKernelGGL(fill_kernel<float>, dim3(4096), dim3(256), 0, 0, static_cast<float*>(d),
                       st.R * sizes[i], 77u + i, 2e-3f, false);
    segs.push_back(ts_segment{d, sizes[i], col, sizes[i]});
    col += sizes[i];
  }
  SWEEP_CHECK(hipDeviceSynchronize());
  std::vector<Variant> v;
  v.push_back({"dense (production)", [&st] { return dense<Base>(st, 5); }, {}});
  add_segment<Base, decltype(st), 64, 1>(v, st, segs);
  add_segment<Base, decltype(st), 64, 2>(v, st, segs);
  add_segment<Base, decltype(st), 128, 1>(v, st, segs);
  add_segment<Base, decltype(st), 128, 2>(v, st, segs);
  time_variants(v, double(st.active) * st.T_ * 28, 3);
}

#define SWEEP_STR2(x) #x
#define SWEEP_STR(x) SWEEP_STR2(x)
#ifdef SWEEP_FAMILY
constexpr const char* kOnly = SWEEP_STR(SWEEP_FAMILY);
#else
constexpr const char* kOnly = "";
#endif

// True when the build includes family `name` (all, or the SWEEP_FAMILY one).
constexpr bool has(const char* name) {
  const char* a = kOnly;
  if (*a == '\0') return true;
  while (*a != '\0' && *a == *name) {
    ++a;
    ++name;
  }
  return *a == '\0' && *name == '\0';
}

}  // namespace

// Runs the family when this build includes it (inside a template, so a
// family left out of the build is never instantiated).
template <bool ON, typename P, int NS>
bool run_stream(int nh, int bytes_per_elem) {
  if constexpr (ON) {
    stream_family<P, NS>(nh, bytes_per_elem);
    return true;
  } else {
    return false;
  }
}
template <bool ON, typename P, int NS>
bool run_math(int nh, int bytes_per_elem) {
  if constexpr (ON) {
    math_family<P, NS>(nh, bytes_per_elem);
    return true;
  } else {
    return false;
  }
}
template <bool ON>
bool run_segment() {
  if constexpr (ON) {
    segment_family();
    return true;
  } else {
    return false;
  }
}

int main(int argc, char** argv) {
  const std::string fam = argc > 1 ? argv[1] : "";
  const std::string cfg = argc > 2 ? argv[2] : "cfg5";
  if (cfg == "cfg2") {
    g_work = Workload{100, 265484, 75};
  } else if (cfg == "cfg4") {
    g_work = Workload{64, 545100, 100};
  } else if (cfg != "cfg5") {
    long r = 0, t = 0;
    int pct = 0;
    if (sscanf(cfg.c_str(), "%ldx%ldx%d", &r, &t, &pct) != 3 || r <= 0 || t <= 0 || t % 4 != 0 ||
        pct <= 0 || pct > 100) {
      fprintf(stderr, "unknown workload '%s' (cfg2, cfg4, cfg5 or RxTxPCT, T a multiple of 4)\n",
              cfg.c_str());
      return 2;
    }
    g_work = Workload{r, t, pct};
  }
  if (fam == "seg_adam_f32" && cfg != "cfg5") {
    fprintf(stderr, "the segmented family has config 5's layout only\n");
    return 2;
  }
  printf("shape_sweep %s %s: R=%ld T=%ld\n", fam.c_str(), cfg.c_str(),
         static_cast<long>(g_work.R), static_cast<long>(g_work.T));
  bool ran = false;
#define SWEEP_STREAM(NAME, NS, NH, BYTES, ...) \
  else if (fam == #NAME) ran = run_stream<has(#NAME), __VA_ARGS__, NS>(NH, BYTES);
  if (false) {
  }
  SWEEP_STREAM(adam_f32, 2, 5, 28, AdamPolicy<float, false, false>)
  SWEEP_STREAM(adam_ams_f32, 3, 5, 36, AdamPolicy<float, false, true>)
  SWEEP_STREAM(adam_bf16state, 2, 5, 20, AdamPolicy<float, false, false, bf16_t>)
  SWEEP_STREAM(adam_f16, 2, 5, 14, AdamPolicy<_Float16, false, false>)
  SWEEP_STREAM(adam_bf16, 2, 5, 14, AdamPolicy<bf16_t, false, false>)
  SWEEP_STREAM(sgd_f32, 1, 4, 20, SgdPolicy<float, true, false>)
  SWEEP_STREAM(sgd_bf16state, 1, 4, 16, SgdPolicy<float, true, false, bf16_t>)
  SWEEP_STREAM(sgd_f16, 1, 4, 10, SgdPolicy<_Float16, true, false>)
  SWEEP_STREAM(sgd_bf16, 1, 4, 10, SgdPolicy<bf16_t, true, false>)
  SWEEP_STREAM(adagrad_f32, 1, 4, 20, AdagradPolicy<float>)
  SWEEP_STREAM(adagrad_bf16state, 1, 4, 16, AdagradPolicy<float, bf16_t>)
  SWEEP_STREAM(adagrad_f16, 1, 4, 10, AdagradPolicy<_Float16>)
  SWEEP_STREAM(adagrad_bf16, 1, 4, 10, AdagradPolicy<bf16_t>)
#define SWEEP_MATH(NAME, NS, NH, BYTES, ...) \
  else if (fam == #NAME) ran = run_math<has(#NAME), __VA_ARGS__, NS>(NH, BYTES);
  SWEEP_MATH(math_adam_f32, 2, 5, 28, AdamPolicy<float, false, false>)
  SWEEP_MATH(math_adam_bf16state, 2, 5, 20, AdamPolicy<float, false, false, bf16_t>)
  SWEEP_MATH(math_adam_f16, 2, 5, 14, AdamPolicy<_Float16, false, false>)
  SWEEP_MATH(math_adam_bf16, 2, 5, 14, AdamPolicy<bf16_t, false, false>)
  SWEEP_MATH(math_adagrad_f32, 1, 4, 20, AdagradPolicy<float>)
  SWEEP_MATH(math_adagrad_f16, 1, 4, 10, AdagradPolicy<_Float16>)
  SWEEP_MATH(math_adagrad_bf16, 1, 4, 10, AdagradPolicy<bf16_t>)
#undef SWEEP_MATH
  else if (fam == "seg_adam_f32") ran = run_segment<has("seg_adam_f32")>();
  else {
    fprintf(stderr, "unknown family '%s'\n", fam.c_str());
    return 2;
  }
#undef SWEEP_STREAM
  if (!ran) {
    fprintf(stderr, "family '%s' not in this build (SWEEP_FAMILY=%s)\n", fam.c_str(), kOnly);
    return 2;
  }
  return 0;
}
