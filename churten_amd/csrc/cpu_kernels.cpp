// cpu_kernels.cpp -- the CPU dispatch key of the torchstrap operators.
//
// CPU tensors are served here; GPU tensors never are (the dispatcher routes by
// device and the GPU key goes to the HIP kernels). The results must be the
// reference CPU kernels' results bit for bit (src/torchstrap/kernels/csrc/cpu/
// {adam,sgd,adagrad}.cpp, built for AVX2), since that is what a torchstrap user
// on CPU gets today. Those kernels have two element formulations per optimizer:
// an 8-lane AVX2 vector body (4 lanes for fp64) and a scalar form used for the
// last T % lanes elements of each row and for every element of a strided
// layout; they differ in where a multiply is fused into an add. The functions
// below state each formulation per element with explicit fma() calls, and this
// file is compiled with -ffp-contract=off, so the rounding sequence is fixed by
// the source; the compiler is free to vectorise the element loops, which does
// not change any result.
//
// Work split as the reference's (cpu/consolidated.h:26-51): (replica, chunk)
// tasks over torch's intra-op thread pool, frozen replicas skipped outright,
// per-replica constants computed in double then narrowed where the reference
// narrows them (cpu/adam.cpp:333-358, sgd.cpp:244-268, adagrad.cpp:207-218).

#include <ATen/ATen.h>
#include <ATen/Dispatch.h>
#include <ATen/Parallel.h>
#include <c10/util/BFloat16.h>
#include <c10/util/Half.h>
#include <torch/library.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <optional>
#include <type_traits>

namespace churten {
namespace cpu {
namespace {

constexpr int64_t kChunk = 16384;

template <typename T> struct math_type { using type = float; };
template <> struct math_type<double> { using type = double; };
template <typename T> using math_t = typename math_type<T>::type;

// Lanes of the reference's vector body: 8 floats / 4 doubles (AVX2); 16-bit
// parameters never take it.
template <typename T> constexpr int64_t lanes() {
  return std::is_same<T, float>::value ? 8 : (std::is_same<T, double>::value ? 4 : 0);
}

template <typename F>
void for_chunks(int64_t R, int64_t T, const bool* mask, F&& fn) {
  const int64_t n_chunks = (T + kChunk - 1) / kChunk;
  at::parallel_for(0, R * n_chunks, 1, [&](int64_t begin, int64_t end) {
    for (int64_t i = begin; i < end; ++i) {
      const int64_t r = i / n_chunks;
      if (!mask[r]) continue;
      const int64_t off = (i % n_chunks) * kChunk;
      fn(r, off, std::min(kChunk, T - off));
    }
  });
}

struct View {
  int64_t sr, st;
};

// Turns a runtime flag into a compile-time one, so the element loops carry no
// per-element branches and vectorise cleanly.
template <typename F>
inline void with_flag(bool b, F&& f) {
  if (b) f(std::true_type{});
  else f(std::false_type{});
}

template <typename T>
View view_of(const at::Tensor& t) {
  return View{t.stride(0), t.stride(1)};
}

// x86 maxps as ATen's vector `maximum` uses it: NaN in -> all-ones NaN out.
template <typename M>
inline M vec_maximum(M a, M b) {
  if (std::isnan(a) || std::isnan(b)) {
    if constexpr (std::is_same<M, float>::value) {
      uint32_t bits = 0xFFFFFFFFu;
      float f;
      std::memcpy(&f, &bits, 4);
      return f;
    } else {
      uint64_t bits = ~uint64_t(0);
      double d;
      std::memcpy(&d, &bits, 8);
      return d;
    }
  }
  return a > b ? a : b;
}

// ===========================================================================
// Adam / AdamW (cpu/adam.cpp:131-270)
// ===========================================================================
template <typename M>
struct AdamC {
  M step_size, beta2, c1, c2, bc2s, eps, wd, wd_mul;
  bool has_wd, lerp_small, maximize;
};

template <typename M>
AdamC<M> adam_consts(double lr, double b1, double b2, double eps, double wd,
                     double step, bool maximize) {
  const double bc1 = 1 - std::pow(b1, step);
  const double bc2 = 1 - std::pow(b2, step);
  AdamC<M> c;
  c.step_size = static_cast<M>(lr / bc1);
  c.beta2 = static_cast<M>(b2);
  c.c1 = static_cast<M>(1 - b1);
  c.c2 = static_cast<M>(1 - b2);
  c.bc2s = static_cast<M>(std::sqrt(bc2));
  c.eps = static_cast<M>(eps);
  c.wd = static_cast<M>(wd);
  c.wd_mul = static_cast<M>(std::fma(-lr, wd, 1.0));  // 1 - lr*wd, fused
  c.has_wd = wd != 0.0;
  c.lerp_small = std::abs(c.c1) < M(0.5);
  c.maximize = maximize;
  return c;
}

// Vector-body element.
template <typename M, bool AMS, bool ADAMW, bool MAX, bool WD, bool LERP_SMALL>
inline void adam_vec_elem(M& p, M g, M& m, M& v, M& mx, const AdamC<M>& c) {
  if (MAX) g = g * M(-1);
  if (WD) {
    if (ADAMW) p = p * c.wd_mul;
    else g = std::fma(p, c.wd, g);
  }
  const M coeff = LERP_SMALL ? c.c1 : c.c1 - M(1);
  const M base = LERP_SMALL ? m : g;
  m = std::fma(coeff, g - m, base);
  v = std::fma(c.c2 * g, g, v * c.beta2);
  M denom;
  if (AMS) {
    mx = vec_maximum(mx, v);
    denom = std::sqrt(mx) / c.bc2s + c.eps;
  } else {
    denom = std::sqrt(v) / c.bc2s + c.eps;
  }
  p = p + ((-c.step_size) * m) / denom;
}

// Scalar element (row tail and strided layouts).
template <typename M, bool AMS, bool ADAMW>
inline void adam_scalar_elem(M& p, M g, M& m, M& v, M& mx, const AdamC<M>& c) {
  if (c.maximize) g = -g;
  if (c.has_wd) {
    if (ADAMW) p = p * c.wd_mul;
    else g = std::fma(p, c.wd, g);
  }
  if (c.lerp_small) m = std::fma(c.c1, g - m, m);
  else m = std::fma(-(g - m), M(1) - c.c1, g);
  v = std::fma(v, c.beta2, (c.c2 * g) * g);
  M denom;
  if (AMS) {
    mx = mx < v ? v : mx;
    denom = std::sqrt(mx) / c.bc2s + c.eps;
  } else {
    denom = std::sqrt(v) / c.bc2s + c.eps;
  }
  p = p - (c.step_size * m) / denom;
}

template <typename T, bool AMS, bool ADAMW>
void adam_run(at::Tensor& params, const at::Tensor& grads, at::Tensor& m_t,
              at::Tensor& v_t, at::Tensor* mx_t, const at::Tensor& steps,
              const at::Tensor& lr, const at::Tensor& b1, const at::Tensor& b2,
              const at::Tensor& eps, const at::Tensor& wd, const at::Tensor& mask,
              bool maximize) {
  using M = math_t<T>;
  const int64_t R = params.size(0), T_ = params.size(1);
  T* P = params.data_ptr<T>();
  const T* G = grads.const_data_ptr<T>();
  T* Mm = m_t.data_ptr<T>();
  T* V = v_t.data_ptr<T>();
  T* X = AMS ? mx_t->data_ptr<T>() : nullptr;
  const View vp = view_of<T>(params), vg = view_of<T>(grads), vm = view_of<T>(m_t),
             vv = view_of<T>(v_t), vx = AMS ? view_of<T>(*mx_t) : View{0, 1};
  const bool unit = vp.st == 1 && vg.st == 1 && vm.st == 1 && vv.st == 1 && vx.st == 1;
  constexpr int64_t K = lanes<T>();
  const bool vec = unit && K > 0;
  const T* S = steps.const_data_ptr<T>();
  const T *L = lr.const_data_ptr<T>(), *B1 = b1.const_data_ptr<T>(),
          *B2 = b2.const_data_ptr<T>(), *E = eps.const_data_ptr<T>(),
          *W = wd.const_data_ptr<T>();
  for_chunks(R, T_, mask.const_data_ptr<bool>(), [&](int64_t r, int64_t off, int64_t n) {
    const AdamC<M> c = adam_consts<M>(
        static_cast<double>(L[r]), static_cast<double>(B1[r]), static_cast<double>(B2[r]),
        static_cast<double>(E[r]), static_cast<double>(W[r]), static_cast<double>(S[r]),
        maximize);
    T* p = P + r * vp.sr + off * vp.st;
    const T* g = G + r * vg.sr + off * vg.st;
    T* m = Mm + r * vm.sr + off * vm.st;
    T* v = V + r * vv.sr + off * vv.st;
    T* x = AMS ? X + r * vx.sr + off * vx.st : nullptr;
    const int64_t body = vec ? n - n % K : 0;
    if constexpr (std::is_same<T, M>::value) {
      with_flag(c.maximize, [&](auto MAX) {
        with_flag(c.has_wd, [&](auto WD) {
          with_flag(c.lerp_small, [&](auto LS) {
            for (int64_t i = 0; i < body; ++i) {
              M xi = AMS ? x[i] : M(0);
              adam_vec_elem<M, AMS, ADAMW, MAX(), WD(), LS()>(p[i], g[i], m[i], v[i], xi, c);
              if (AMS) x[i] = xi;
            }
          });
        });
      });
    }
    for (int64_t i = body; i < n; ++i) {
      M pi = static_cast<M>(p[i * vp.st]), mi = static_cast<M>(m[i * vm.st]),
        vi = static_cast<M>(v[i * vv.st]), xi = AMS ? static_cast<M>(x[i * vx.st]) : M(0);
      adam_scalar_elem<M, AMS, ADAMW>(pi, static_cast<M>(g[i * vg.st]), mi, vi, xi, c);
      p[i * vp.st] = static_cast<T>(pi);
      m[i * vm.st] = static_cast<T>(mi);
      v[i * vv.st] = static_cast<T>(vi);
      if (AMS) x[i * vx.st] = static_cast<T>(xi);
    }
  });
}

// ===========================================================================
// SGD (cpu/sgd.cpp:91-283)
// ===========================================================================
template <typename M>
struct SgdC {
  M wd, mom, omd, lr, neg_lr;
  bool has_wd, first, maximize;
};

template <typename M, bool BUF, bool NEST, bool MAX, bool WD, bool FIRST>
inline void sgd_elem(M& p, M g, M& b, const SgdC<M>& c, bool vec) {
  if (MAX) g = vec ? g * M(-1) : -g;
  if (WD) g = std::fma(p, c.wd, g);
  if (BUF) {
    M buf;
    if (FIRST) buf = g;
    else if (vec) buf = std::fma(c.omd, g, b * c.mom);
    else buf = std::fma(b, c.mom, g * c.omd);
    b = buf;
    g = NEST ? std::fma(buf, c.mom, g) : buf;
  }
  p = vec ? std::fma(g, c.neg_lr, p) : std::fma(-g, c.lr, p);
}

template <typename T, bool BUF, bool NEST>
void sgd_run(at::Tensor& params, const at::Tensor& grads, at::Tensor* mb_t,
             const at::Tensor& steps, const at::Tensor& lr, const at::Tensor& mom,
             const at::Tensor& damp, const at::Tensor& wd, const at::Tensor& mask,
             bool maximize) {
  using M = math_t<T>;
  const int64_t R = params.size(0), T_ = params.size(1);
  T* P = params.data_ptr<T>();
  const T* G = grads.const_data_ptr<T>();
  T* B = BUF ? mb_t->data_ptr<T>() : nullptr;
  const View vp = view_of<T>(params), vg = view_of<T>(grads),
             vb = BUF ? view_of<T>(*mb_t) : View{0, 1};
  constexpr int64_t K = lanes<T>();
  const bool vec = vp.st == 1 && vg.st == 1 && vb.st == 1 && K > 0;
  const T *S = steps.const_data_ptr<T>(), *L = lr.const_data_ptr<T>(),
          *MO = mom.const_data_ptr<T>(), *D = damp.const_data_ptr<T>(),
          *W = wd.const_data_ptr<T>();
  for_chunks(R, T_, mask.const_data_ptr<bool>(), [&](int64_t r, int64_t off, int64_t n) {
    const double lr_d = static_cast<double>(L[r]), wd_d = static_cast<double>(W[r]);
    SgdC<M> c;
    c.wd = static_cast<M>(wd_d);
    c.mom = static_cast<M>(static_cast<double>(MO[r]));
    c.omd = static_cast<M>(1 - static_cast<double>(D[r]));
    c.lr = static_cast<M>(lr_d);
    c.neg_lr = static_cast<M>(-lr_d);
    c.has_wd = wd_d != 0.0;
    c.first = static_cast<double>(S[r]) == 1.0;
    c.maximize = maximize;
    T* p = P + r * vp.sr + off * vp.st;
    const T* g = G + r * vg.sr + off * vg.st;
    T* b = BUF ? B + r * vb.sr + off * vb.st : nullptr;
    const int64_t body = vec ? n - n % K : 0;
    with_flag(c.maximize, [&](auto MAX) {
      with_flag(c.has_wd, [&](auto WD) {
        with_flag(c.first, [&](auto FIRST) {
          if constexpr (std::is_same<T, M>::value) {
            for (int64_t i = 0; i < body; ++i) {
              M bi = (BUF && !FIRST()) ? b[i] : M(0);
              sgd_elem<M, BUF, NEST, MAX(), WD(), FIRST()>(p[i], g[i], bi, c, true);
              if (BUF) b[i] = bi;
            }
          }
          for (int64_t i = body; i < n; ++i) {
            M pi = static_cast<M>(p[i * vp.st]);
            M bi = (BUF && !FIRST()) ? static_cast<M>(b[i * vb.st]) : M(0);
            sgd_elem<M, BUF, NEST, MAX(), WD(), FIRST()>(pi, static_cast<M>(g[i * vg.st]), bi,
                                                          c, false);
            p[i * vp.st] = static_cast<T>(pi);
            if (BUF) b[i * vb.st] = static_cast<T>(bi);
          }
        });
      });
    });
  });
}

// ===========================================================================
// Adagrad (cpu/adagrad.cpp:80-233): float element loop, clr in double
// ===========================================================================
template <typename M, bool MAX, bool WD>
inline void adagrad_elem(M& p, M g, M& s, M clr, M wd, M eps, bool vec) {
  if (MAX) g = vec ? g * M(-1) : -g;
  if (WD) g = std::fma(p, wd, g);
  s = std::fma(g, g, s);
  const M denom = std::sqrt(s) + eps;
  p = p - (clr * g) / denom;
}

template <typename T>
void adagrad_run(at::Tensor& params, const at::Tensor& grads, at::Tensor& s_t,
                 const at::Tensor& steps, const at::Tensor& lr, const at::Tensor& lrd,
                 const at::Tensor& wd, const at::Tensor& eps, const at::Tensor& mask,
                 bool maximize) {
  using M = math_t<T>;
  const int64_t R = params.size(0), T_ = params.size(1);
  T* P = params.data_ptr<T>();
  const T* G = grads.const_data_ptr<T>();
  T* Sm = s_t.data_ptr<T>();
  const View vp = view_of<T>(params), vg = view_of<T>(grads), vs = view_of<T>(s_t);
  constexpr int64_t K = lanes<T>();
  const bool vec = vp.st == 1 && vg.st == 1 && vs.st == 1 && K > 0;
  const T *ST = steps.const_data_ptr<T>(), *L = lr.const_data_ptr<T>(),
          *LD = lrd.const_data_ptr<T>(), *W = wd.const_data_ptr<T>(),
          *E = eps.const_data_ptr<T>();
  for_chunks(R, T_, mask.const_data_ptr<bool>(), [&](int64_t r, int64_t off, int64_t n) {
    const double step = static_cast<double>(ST[r]);
    const double clr_d = static_cast<double>(L[r]) /
                         std::fma(step - 1.0, static_cast<double>(LD[r]), 1.0);
    const M clr = static_cast<M>(clr_d);
    const M wdm = static_cast<M>(static_cast<double>(W[r]));
    const M em = static_cast<M>(static_cast<double>(E[r]));
    const bool has_wd = static_cast<double>(W[r]) != 0.0;
    T* p = P + r * vp.sr + off * vp.st;
    const T* g = G + r * vg.sr + off * vg.st;
    T* s = Sm + r * vs.sr + off * vs.st;
    const int64_t body = vec ? n - n % K : 0;
    with_flag(maximize, [&](auto MAX) {
      with_flag(has_wd, [&](auto WD) {
        if constexpr (std::is_same<T, M>::value) {
          for (int64_t i = 0; i < body; ++i) {
            adagrad_elem<M, MAX(), WD()>(p[i], g[i], s[i], clr, wdm, em, true);
          }
        }
        for (int64_t i = body; i < n; ++i) {
          M pi = static_cast<M>(p[i * vp.st]), si = static_cast<M>(s[i * vs.st]);
          adagrad_elem<M, MAX(), WD()>(pi, static_cast<M>(g[i * vg.st]), si, clr, wdm, em,
                                       false);
          p[i * vp.st] = static_cast<T>(pi);
          s[i * vs.st] = static_cast<T>(si);
        }
      });
    });
  });
}

// ===========================================================================
// Operator entry points
// ===========================================================================
void check_rt(const at::Tensor& params, const at::Tensor& t, const char* op,
              const char* name) {
  TORCH_CHECK(t.dim() == 2 && t.sizes() == params.sizes(), op, ": ", name,
              " must have params' shape ", params.sizes(), ", got ", t.sizes());
  TORCH_CHECK(t.scalar_type() == params.scalar_type(), op, ": ", name,
              " must have params' dtype ", params.scalar_type());
  TORCH_CHECK(t.device() == params.device(), op, ": ", name, " must be on ",
              params.device());
}

void check_vec(const at::Tensor& params, const at::Tensor& t, const char* op,
               const char* name) {
  TORCH_CHECK(t.numel() == params.size(0), op, ": ", name, " must have R = ",
              params.size(0), " elements (one per replica), got ", t.numel());
  TORCH_CHECK(t.device() == params.device(), op, ": ", name, " must be on ",
              params.device());
}

at::Tensor hyper(const at::Tensor& t, at::ScalarType dtype) {
  return t.reshape({t.numel()}).to(dtype).contiguous();
}

at::Tensor mask_of(const at::Tensor& m) {
  return m.reshape({m.numel()}).to(at::kBool).contiguous();
}

// bfloat16 optimizer state next to float32 params (an extension; the
// reference rejects mixed dtypes): the float32 kernel runs on widened copies of
// the state, which is then rounded back to nearest-even bfloat16.
bool bf16_state(const at::Tensor& params, const at::Tensor& state) {
  return params.scalar_type() == at::kFloat && state.scalar_type() == at::kBFloat16;
}

// A float32 working copy of bfloat16 state, always row-major: whether a row
// takes the vector formulation then depends on the params' and grads' layout
// only, not on how the bfloat16 buffer happens to be stored.
at::Tensor widen(const at::Tensor& state) {
  return state.to(at::kFloat, false, false, at::MemoryFormat::Contiguous);
}

// Rounds the active rows of a widened state copy back into the bfloat16
// buffer; frozen rows keep their bits.
void store_active_rows(at::Tensor& dst, const at::Tensor& src, const at::Tensor& active_mask) {
  const at::Tensor rows = active_mask.reshape({-1}).to(at::kBool).nonzero().reshape({-1});
  dst.index_copy_(0, rows, src.index_select(0, rows).to(dst.scalar_type()));
}

void check_bf16_state(const at::Tensor& params, const at::Tensor& t, const char* op,
                      const char* name) {
  TORCH_CHECK(t.dim() == 2 && t.sizes() == params.sizes(), op, ": ", name,
              " must have params' shape ", params.sizes(), ", got ", t.sizes());
  TORCH_CHECK(t.scalar_type() == at::kBFloat16, op, ": ", name,
              " must be bfloat16 like the other state buffers");
  TORCH_CHECK(t.device() == params.device(), op, ": ", name, " must be on ",
              params.device());
}

at::Tensor adam_step_cpu(at::Tensor params, at::Tensor grads, at::Tensor exp_avgs,
                         at::Tensor exp_avg_sqs, std::optional<at::Tensor> max_exp_avg_sqs,
                         at::Tensor state_steps, at::Tensor lr, at::Tensor beta1,
                         at::Tensor beta2, at::Tensor eps, at::Tensor weight_decay,
                         at::Tensor active_mask, bool amsgrad, bool maximize,
                         bool decoupled_weight_decay) {
  constexpr const char* op = "torchstrap::adam_step_";
  TORCH_CHECK(params.dim() == 2, op, ": params must be a 2-D (R, T) buffer");
  TORCH_CHECK(!amsgrad || max_exp_avg_sqs.has_value(), "amsgrad=True requires max_exp_avg_sqs");
  if (bf16_state(params, exp_avgs)) {
    check_bf16_state(params, exp_avgs, op, "exp_avgs");
    check_bf16_state(params, exp_avg_sqs, op, "exp_avg_sqs");
    if (amsgrad) check_bf16_state(params, *max_exp_avg_sqs, op, "max_exp_avg_sqs");
    at::Tensor m = widen(exp_avgs), v = widen(exp_avg_sqs);
    std::optional<at::Tensor> mx;
    if (amsgrad) mx = widen(*max_exp_avg_sqs);
    at::Tensor out = adam_step_cpu(params, grads, m, v, mx, state_steps, lr, beta1, beta2, eps,
                                   weight_decay, active_mask, amsgrad, maximize,
                                   decoupled_weight_decay);
    store_active_rows(exp_avgs, m, active_mask);
    store_active_rows(exp_avg_sqs, v, active_mask);
    if (amsgrad) store_active_rows(*max_exp_avg_sqs, *mx, active_mask);
    return out;
  }
  check_rt(params, grads, op, "grads");
  check_rt(params, exp_avgs, op, "exp_avgs");
  check_rt(params, exp_avg_sqs, op, "exp_avg_sqs");
  if (amsgrad) check_rt(params, *max_exp_avg_sqs, op, "max_exp_avg_sqs");
  for (auto* p : {&state_steps, &lr, &beta1, &beta2, &eps, &weight_decay, &active_mask})
    check_vec(params, *p, op, "a per-replica input");
  state_steps.add_(active_mask.to(state_steps.scalar_type()));
  if (params.size(0) == 0 || params.size(1) == 0) return at::zeros({}, params.options());
  const auto dt = params.scalar_type();
  const auto st = hyper(state_steps, dt), l = hyper(lr, dt), b1 = hyper(beta1, dt),
             b2 = hyper(beta2, dt), e = hyper(eps, dt), w = hyper(weight_decay, dt);
  const auto mk = mask_of(active_mask);
  at::Tensor* mx = amsgrad ? &*max_exp_avg_sqs : nullptr;
  AT_DISPATCH_FLOATING_TYPES_AND2(at::kHalf, at::kBFloat16, dt, "adam_step_cpu", [&] {
    if (amsgrad) {
      if (decoupled_weight_decay)
        adam_run<scalar_t, true, true>(params, grads, exp_avgs, exp_avg_sqs, mx, st, l, b1, b2, e, w, mk, maximize);
      else
        adam_run<scalar_t, true, false>(params, grads, exp_avgs, exp_avg_sqs, mx, st, l, b1, b2, e, w, mk, maximize);
    } else {
      if (decoupled_weight_decay)
        adam_run<scalar_t, false, true>(params, grads, exp_avgs, exp_avg_sqs, mx, st, l, b1, b2, e, w, mk, maximize);
      else
        adam_run<scalar_t, false, false>(params, grads, exp_avgs, exp_avg_sqs, mx, st, l, b1, b2, e, w, mk, maximize);
    }
  });
  return at::zeros({}, params.options());
}

at::Tensor sgd_step_cpu(at::Tensor params, at::Tensor grads,
                        std::optional<at::Tensor> momentum_buffers, at::Tensor state_steps,
                        at::Tensor lr, at::Tensor momentum, at::Tensor dampening,
                        at::Tensor weight_decay, at::Tensor active_mask, bool nesterov,
                        bool maximize) {
  constexpr const char* op = "torchstrap::sgd_step_";
  TORCH_CHECK(params.dim() == 2, op, ": params must be a 2-D (R, T) buffer");
  TORCH_CHECK(!nesterov || momentum_buffers.has_value(), "nesterov=True requires momentum_buffers");
  if (momentum_buffers.has_value() && bf16_state(params, *momentum_buffers)) {
    check_bf16_state(params, *momentum_buffers, op, "momentum_buffers");
    std::optional<at::Tensor> mb = widen(*momentum_buffers);
    at::Tensor out = sgd_step_cpu(params, grads, mb, state_steps, lr, momentum, dampening,
                                  weight_decay, active_mask, nesterov, maximize);
    store_active_rows(*momentum_buffers, *mb, active_mask);
    return out;
  }
  check_rt(params, grads, op, "grads");
  const bool has_buf = momentum_buffers.has_value();
  if (has_buf) check_rt(params, *momentum_buffers, op, "momentum_buffers");
  for (auto* p : {&state_steps, &lr, &momentum, &dampening, &weight_decay, &active_mask})
    check_vec(params, *p, op, "a per-replica input");
  state_steps.add_(active_mask.to(state_steps.scalar_type()));
  if (params.size(0) == 0 || params.size(1) == 0) return at::zeros({}, params.options());
  const auto dt = params.scalar_type();
  const auto st = hyper(state_steps, dt), l = hyper(lr, dt), mo = hyper(momentum, dt),
             d = hyper(dampening, dt), w = hyper(weight_decay, dt);
  const auto mk = mask_of(active_mask);
  at::Tensor* mb = has_buf ? &*momentum_buffers : nullptr;
  AT_DISPATCH_FLOATING_TYPES_AND2(at::kHalf, at::kBFloat16, dt, "sgd_step_cpu", [&] {
    if (has_buf) {
      if (nesterov) sgd_run<scalar_t, true, true>(params, grads, mb, st, l, mo, d, w, mk, maximize);
      else sgd_run<scalar_t, true, false>(params, grads, mb, st, l, mo, d, w, mk, maximize);
    } else {
      sgd_run<scalar_t, false, false>(params, grads, mb, st, l, mo, d, w, mk, maximize);
    }
  });
  return at::zeros({}, params.options());
}

at::Tensor adagrad_step_cpu(at::Tensor params, at::Tensor grads, at::Tensor state_sums,
                            at::Tensor state_steps, at::Tensor lr, at::Tensor lr_decay,
                            at::Tensor weight_decay, at::Tensor eps, at::Tensor active_mask,
                            bool maximize) {
  constexpr const char* op = "torchstrap::adagrad_step_";
  TORCH_CHECK(params.dim() == 2, op, ": params must be a 2-D (R, T) buffer");
  if (bf16_state(params, state_sums)) {
    check_bf16_state(params, state_sums, op, "state_sums");
    at::Tensor s32 = widen(state_sums);
    at::Tensor out = adagrad_step_cpu(params, grads, s32, state_steps, lr, lr_decay,
                                      weight_decay, eps, active_mask, maximize);
    store_active_rows(state_sums, s32, active_mask);
    return out;
  }
  check_rt(params, grads, op, "grads");
  check_rt(params, state_sums, op, "state_sums");
  for (auto* p : {&state_steps, &lr, &lr_decay, &weight_decay, &eps, &active_mask})
    check_vec(params, *p, op, "a per-replica input");
  state_steps.add_(active_mask.to(state_steps.scalar_type()));
  if (params.size(0) == 0 || params.size(1) == 0) return at::zeros({}, params.options());
  const auto dt = params.scalar_type();
  const auto st = hyper(state_steps, dt), l = hyper(lr, dt), ld = hyper(lr_decay, dt),
             w = hyper(weight_decay, dt), e = hyper(eps, dt);
  const auto mk = mask_of(active_mask);
  AT_DISPATCH_FLOATING_TYPES_AND2(at::kHalf, at::kBFloat16, dt, "adagrad_step_cpu", [&] {
    adagrad_run<scalar_t>(params, grads, state_sums, st, l, ld, w, e, mk, maximize);
  });
  return at::zeros({}, params.options());
}

}  // namespace

TORCH_LIBRARY_IMPL(torchstrap, CPU, m) {
  m.impl("adam_step_", &adam_step_cpu);
  m.impl("sgd_step_", &sgd_step_cpu);
  m.impl("adagrad_step_", &adagrad_step_cpu);
}

}  // namespace cpu
}  // namespace churten
