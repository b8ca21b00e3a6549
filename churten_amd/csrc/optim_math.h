// optim_math.h -- per-element update arithmetic of the three fused optimizers,
// plus the storage-type conversions the kernels need.
//
// Bit-exactness contract. On the MI355X the update of every active replica must
// be bit-identical to torch's own ROCm fused kernels (`torch._fused_adam_`,
// `_fused_adamw_`, `_fused_sgd_`, `_fused_adagrad_`). The reference gets that on
// its GPU by calling ATen's device math verbatim (src/torchstrap/kernels/csrc/
// cuda/adam.cu:146-157, cuda/adagrad.cu:141-148) or by transcribing it
// (cuda/sgd.cu:90-132). This file restates the same arithmetic: the order of the
// operations, the type each intermediate is held in (float vs double) and the
// point where a double is narrowed to float are the algorithm, so they follow the
// ROCm headers shipped with torch 2.10.0+rocm7.0:
//   torch/include/ATen/native/hip/fused_adam_utils.cuh:28-92   (adam_math)
//   torch/include/ATen/native/hip/fused_adam_utils.cuh:131-139 (bias corrections)
//   torch/include/ATen/native/hip/fused_adagrad_utils.cuh:16-50, 75-81
// torch compiles those headers with hipcc's default -ffp-contract=fast, so
// each `a * b + c` there is one fused multiply-add. Here every such
// contraction is written out as an explicit fma in the order torch's build
// fuses it (the order the parity tests pin on the GPU), so
// the result does not depend on which kernel the math is inlined into or on
// what the compiler decides there. Float division and sqrt are IEEE correctly
// rounded (hipcc's default). Each function is checked bit-for-bit against
// torch on the GPU.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace churten {

// ---------------------------------------------------------------------------
// Storage types. fp16 is clang's _Float16; bf16 is carried as raw bits with
// c10::BFloat16's conversions (widen = shift, narrow = round to nearest even,
// NaN -> quiet NaN).
// ---------------------------------------------------------------------------
struct bf16_t {
  uint16_t bits;
};

template <typename T> struct op_type { using type = float; };
template <> struct op_type<double> { using type = double; };
template <typename T> using op_t = typename op_type<T>::type;

__device__ __forceinline__ float widen(float x) { return x; }
__device__ __forceinline__ double widen(double x) { return x; }
__device__ __forceinline__ float widen(_Float16 x) { return static_cast<float>(x); }
__device__ __forceinline__ float widen(bf16_t x) {
  return __uint_as_float(static_cast<uint32_t>(x.bits) << 16);
}

template <typename T> __device__ __forceinline__ T narrow(op_t<T> x);
template <> __device__ __forceinline__ float narrow<float>(float x) { return x; }
template <> __device__ __forceinline__ double narrow<double>(double x) { return x; }
// The float value itself is rounded to half. torch narrows in two steps
// (double expression -> float opmath value -> half on store); hipcc's default
// -ffp-contract=fast lets the backend fold such a double -> float -> half chain
// into one double -> half rounding, which differs whenever the float lands on
// a half-way point between two halves. The empty asm makes the float opaque,
// so both roundings happen.
template <> __device__ __forceinline__ _Float16 narrow<_Float16>(float x) {
  asm("" : "+v"(x));
  return static_cast<_Float16>(x);
}
// Round to nearest even, as torch's float -> bfloat16: gfx950 converts in
// hardware (v_cvt_pk_bf16_f32); NaN becomes torch's canonical 0x7FC0. The
// empty asm keeps the float rounding of the value, as for half.
template <> __device__ __forceinline__ bf16_t narrow<bf16_t>(float x) {
  asm("" : "+v"(x));
  bf16_t out;
  out.bits = x != x ? static_cast<uint16_t>(0x7FC0u)
                    : __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
  return out;
}

// a * b + c rounded once, to half (v_fma_mixlo_f16 on float operands: the
// exact value, one rounding to nearest even, half subnormals kept), returned
// as the float holding that half, which narrow<_Float16> passes unchanged.
// Rounding the float fma to half instead rounds twice, and differs where the
// float result is a half-way point between two halves and the exact one is not.
__device__ __forceinline__ float fma_half(float a, float b, float c) {
  uint32_t d = 0;
  asm("v_fma_mixlo_f16 %0, %1, %2, %3" : "+v"(d) : "v"(a), "v"(b), "v"(c));
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(d)));
}

// The pair (a0 * a0 + c.lo, a1 * a1 + c.hi) for float a0, a1 and a packed
// pair of halves c (as loaded), each rounded once to half as fma_half, packed
// the same way: v_fma_mixlo_f16 writes the low half, v_fma_mixhi_f16 the high
// half of the same register, and op_sel picks c's half as an f16 operand (no
// conversion of c).
__device__ __forceinline__ uint32_t fma_half2_sq(float a0, float a1, uint32_t c) {
  uint32_t d;
  asm("v_fma_mixlo_f16 %0, %1, %1, %3 op_sel_hi:[0,0,1]\n\t"
      "v_fma_mixhi_f16 %0, %2, %2, %3 op_sel:[0,0,1] op_sel_hi:[0,0,1]"
      : "=&v"(d)
      : "v"(a0), "v"(a1), "v"(c));
  return d;
}

// Two floats to a packed pair of bfloat16 (first in the low half), each exactly
// as narrow<bf16_t>: one v_cvt_pk_bf16_f32 for both, with NaN made torch's
// 0x7FC0 on the float side (the conversion keeps a quiet NaN's top bits, and
// 0x7FC00000 has none below them). One instruction per value fewer than two
// separate narrowings and the packing.
__device__ __forceinline__ uint32_t narrow2_bf16(float a, float b) {
  asm("" : "+v"(a), "+v"(b));
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  a = a != a ? __uint_as_float(0x7FC00000u) : a;
  b = b != b ? __uint_as_float(0x7FC00000u) : b;
  const f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// Correctly rounded float square root, bit-identical to std::sqrt as hipcc
// expands it: v_sqrt_f32 (within an ulp), then one correction step that
// compares x with the products of the result and its two neighbours. The
// expansion first scales x < 2^-96 by 2^32 (so the correction's residuals stay
// exact) and returns +-0 and +inf as themselves. For x >= 2^-96, +inf and NaN
// the scaling and the special-case select are no-ops (for +inf the correction
// keeps +inf; NaN stays v_sqrt's NaN), so sqrt_rn_short drops them: 9 VALU
// instructions instead of 16. sqrt_rn takes it when no lane of the wavefront
// holds a tiny, zero or negative x (a wave-uniform branch per value), and
// std::sqrt otherwise. +-0 needs no scaling either: v_sqrt returns it, below
// is a NaN pattern (0xFFFFFFFF / 0x7FFFFFFF, so the first test fails) and the
// residual with above is a zero (not > 0), so the short path returns +-0 as
// std::sqrt does. With ZEROS (the float16-state policies, whose moments
// underflow to zero for small gradients) a wavefront whose only small values
// are zeros takes it too: a second ballot, only when the first finds a small
// value. Elsewhere the single ballot: the second one's few scalar
// instructions per value cost the float32 update about 0.4%. Checked against
// torch's sqrt on every float bit pattern and on wavefronts mixing zeros,
// tiny and ordinary values, both forms.
// Measured against std::sqrt at the config-5 shape (same process, 5 rounds,
// two boxes): Adam with bfloat16 params +2.9-3.6%, Adagrad with half /
// bfloat16 params +4.4-5% / +3.8-3.9%, Adam with half params -0.6 to +0.5%,
// float32 unchanged; one decision per pack of values instead of per value was
// slower for half (-1.6%) and for 16-bit Adagrad.
__device__ __forceinline__ bool sqrt_short_ok(float x) { return !(x < 0x1p-96f); }
__device__ __forceinline__ float sqrt_rn_short(float x) {
  const float s = __builtin_amdgcn_sqrtf(x);
  const float below = __uint_as_float(__float_as_uint(s) - 1u);
  const float above = __uint_as_float(__float_as_uint(s) + 1u);
  const float r_below = __builtin_fmaf(-below, s, x);
  const float r_above = __builtin_fmaf(-above, s, x);
  float r = r_below <= 0.0f ? below : s;
  r = r_above > 0.0f ? above : r;
  return r;
}
template <bool ZEROS = false>
__device__ __forceinline__ float sqrt_rn(float x) {
  if (__ballot(!sqrt_short_ok(x)) != 0) {
    if constexpr (ZEROS) {
      // The zero test stays in this rare branch: computed from an opaque
      // copy, the compiler cannot hoist it into the common path (where it
      // cost three instructions per value).
      float y = x;
      asm volatile("" : "+v"(y));
      if (__ballot(!sqrt_short_ok(y) && y != 0.0f) == 0) {
        return sqrt_rn_short(x);
      }
    }
    return std::sqrt(x);
  }
  return sqrt_rn_short(x);
}
template <bool ZEROS = false>
__device__ __forceinline__ double sqrt_rn(double x) { return std::sqrt(x); }

// ---------------------------------------------------------------------------
// Adam / AdamW. Hyperparameters are doubles (ATen passes them as
// `const double&`), so the moment updates and the weight-decay terms are fp64
// expressions narrowed once to the math type; the bias corrections arrive
// already narrowed to the math type, as ATen's call narrows them.
// ---------------------------------------------------------------------------
struct AdamHyper {
  double lr, beta1, beta2, weight_decay, eps;
};

// A float divided by a per-replica constant b, as a multiply by the double
// `rcp` = RN64(1 / b): RN32(RN64(x * rcp)) == RN32(x / b) bit for bit for
// every float x and b whose quotient is not a subnormal float (zeros,
// infinities and NaNs included; rcp is +-inf for b = +-0 and +-0 for
// b = +-inf), except when x and b are both NaN: then both are NaN, the divide
// with x's payload, the product with b's (for Adam, b is NaN only for a beta2
// that makes 1 - beta2^step negative or NaN). Why: x and b have 24-bit
// significands, so a normal quotient is never a midpoint between two floats (a
// midpoint there has a 25-bit odd significand M, and x = b * M would need M to
// divide x's significand), and its distance to the nearest midpoint is more
// than 2^-49 of |x / b|; the double product errs by at most
// (1 + 2^-53)^2 - 1 < 2^-52 of it, so both sit on the same side of every
// rounding boundary. A subnormal quotient has fewer significant bits, can be an
// exact midpoint, and then the product may round the tie the other way
// (x = 0x00012600, b = 50176: the divide gives 2 * 2^-149, the product
// 2^-149). For Adam x = sqrt(v) of a float v is 0, at least 2^-75, inf or NaN,
// so a subnormal quotient needs b > 2^51, i.e. 1 - beta2^step > 2^102, which
// needs |beta2| > 1 (torch.optim rejects beta2 outside [0, 1)). Nine VALU
// instructions fewer per element than the correctly rounded float divide;
// tests check the identity bit for bit on every float x for a set of b, show
// that the only exceptions are subnormal ties, and check the update against
// torch.
__device__ __forceinline__ float div_by_rcp(float x, double rcp) {
  return static_cast<float>(static_cast<double>(x) * rcp);
}

// Adam's per-replica constants as the element update consumes them: the step
// size lr / bias_correction1 (a double divide narrowed to the math type, as
// ATen writes it) and the divisor of sqrt(v): for float math the reciprocal of
// bias_correction2_sqrt in double (div_by_rcp), for double math the value
// itself.
template <typename opmath_t>
struct AdamConsts {
  opmath_t step_size;
  double bc2s_div;
};

template <typename opmath_t>
__device__ __forceinline__ AdamConsts<opmath_t> adam_consts(
    const double lr, const opmath_t bias_correction1, const opmath_t bias_correction2_sqrt) {
  AdamConsts<opmath_t> c;
  c.step_size = static_cast<opmath_t>(lr / bias_correction1);
  if constexpr (std::is_same<opmath_t, float>::value) {
    c.bc2s_div = 1.0 / static_cast<double>(bias_correction2_sqrt);
  } else {
    c.bc2s_div = bias_correction2_sqrt;
  }
  return c;
}

// sqrt(v) / bias_correction2_sqrt in the math type.
__device__ __forceinline__ float adam_div_bc2s(float s, double d) { return div_by_rcp(s, d); }
__device__ __forceinline__ double adam_div_bc2s(double s, double d) { return s / d; }

// ATen's `x + eps` with eps a double (x the float quotient above), narrowed to
// the float math type. eps holds a float value here (the hyperparameter
// tensors are float, or half / bfloat16, widened), and for two floats the sum
// rounded to double and then to float equals the sum rounded to float once:
// double rounding is harmless for addition because 53 >= 2 * 24 + 1 bits. So
// one float add gives ATen's bits (two fp64-unit instructions fewer); tests
// check the identity on every float x for a set of eps.
__device__ __forceinline__ float adam_add_eps(float x, double eps) {
  return x + static_cast<float>(eps);
}
__device__ __forceinline__ double adam_add_eps(double x, double eps) { return x + eps; }

// The first part of ATen's adam_math for one element: maximize, weight decay,
// the two moments (and the running maximum with amsgrad). Returns the value
// whose square root the denominator takes.
template <typename opmath_t, bool ADAMW, bool AMSGRAD>
__device__ __forceinline__ opmath_t adam_moments(
    opmath_t& param, opmath_t grad, opmath_t& exp_avg, opmath_t& exp_avg_sq,
    opmath_t& max_exp_avg_sq, const AdamHyper& h, const bool maximize) {
  if (maximize) {
    grad = -grad;
  }
  if (h.weight_decay != 0) {
    if constexpr (ADAMW) {
      // param -= lr * weight_decay * param
      param = static_cast<opmath_t>(
          ::fma(-(h.lr * h.weight_decay), double(param), double(param)));
    } else {
      // grad += param * weight_decay
      grad = static_cast<opmath_t>(::fma(double(param), h.weight_decay, double(grad)));
    }
  }
  // exp_avg = beta1 * exp_avg + (1 - beta1) * grad
  exp_avg = static_cast<opmath_t>(
      ::fma(h.beta1, double(exp_avg), (1 - h.beta1) * double(grad)));
  // exp_avg_sq = beta2 * exp_avg_sq + (1 - beta2) * grad * grad
  exp_avg_sq = static_cast<opmath_t>(
      ::fma(h.beta2, double(exp_avg_sq), ((1 - h.beta2) * double(grad)) * double(grad)));
  if constexpr (AMSGRAD) {
    max_exp_avg_sq = ::max(max_exp_avg_sq, exp_avg_sq);
    return max_exp_avg_sq;
  } else {
    return exp_avg_sq;
  }
}

// The rest, given the square root `root` of adam_moments' value. ATen:
// step_size = lr / bias_correction1 (per replica, in c);
// denom = (sqrt(v) / bias_correction2_sqrt) + eps; param -= step_size * m / denom.
template <typename opmath_t>
__device__ __forceinline__ void adam_finish(opmath_t& param, const opmath_t exp_avg,
                                            const opmath_t root, const AdamHyper& h,
                                            const AdamConsts<opmath_t>& c) {
  const opmath_t denom = adam_add_eps(adam_div_bc2s(root, c.bc2s_div), h.eps);
  param -= c.step_size * exp_avg / denom;
}

// One element of ATen's adam_math.
template <typename opmath_t, bool ADAMW, bool AMSGRAD, bool ZEROS = false>
__device__ __forceinline__ void adam_element(
    opmath_t& param, opmath_t grad, opmath_t& exp_avg, opmath_t& exp_avg_sq,
    opmath_t& max_exp_avg_sq, const AdamHyper& h, const bool maximize,
    const AdamConsts<opmath_t>& c) {
  const opmath_t v = adam_moments<opmath_t, ADAMW, AMSGRAD>(param, grad, exp_avg, exp_avg_sq,
                                                            max_exp_avg_sq, h, maximize);
  adam_finish(param, exp_avg, sqrt_rn<ZEROS>(v), h, c);
}

// 1 - beta^step in double, with pow(double, double) from the float step.
__device__ __forceinline__ double adam_bias_correction(const double beta, const float step) {
  return 1 - ::pow(beta, static_cast<double>(step));
}

// Per-replica bias corrections from the (bumped) step count: computed in double
// (adam_bias_correction), then narrowed to the math type.
template <typename opmath_t>
__device__ __forceinline__ void adam_bias_corrections(
    const double beta1, const double beta2, const float step,
    opmath_t& bias_correction1, opmath_t& bias_correction2_sqrt) {
  const double bc1 = adam_bias_correction(beta1, step);
  const double bc2 = adam_bias_correction(beta2, step);
  bias_correction1 = static_cast<opmath_t>(bc1);
  bias_correction2_sqrt = static_cast<opmath_t>(std::sqrt(bc2));
}

// ---------------------------------------------------------------------------
// SGD. `hyper_t` is the type the hyperparameters are carried in inside the
// element math.
// ---------------------------------------------------------------------------
template <typename hyper_t> struct SgdHyper {
  hyper_t weight_decay, momentum, lr, dampening;
};

// Every multiply-add is an explicit fma, in the order torch's ROCm
// `_fused_sgd_` contracts them (pinned on the MI355X for float64 parameters,
// where the products are inexact and the contraction shows: weight decay
// fma(wd, p, g), buffer fma(mom, buf, (1 - damp) * g), Nesterov
// fma(mom, buf, g), update fma(-lr, g, p)). For float32 parameters with
// double hyperparameters the products are exact, so the same code gives the
// same bits as any contraction would. Writing the fmas out keeps the result
// independent of which kernel the element math is inlined into.
template <typename opmath_t, typename hyper_t, bool HAS_BUF, bool NESTEROV>
__device__ __forceinline__ void sgd_element(
    opmath_t& param, opmath_t grad, opmath_t& momentum_buffer,
    const SgdHyper<hyper_t>& h, const bool maximize, const bool is_first_step) {
  using acc_t = decltype(hyper_t() * opmath_t());
  if (maximize) {
    grad *= -1.0;
  }
  if (h.weight_decay != 0) {
    grad = static_cast<opmath_t>(
        ::fma(acc_t(h.weight_decay), acc_t(param), acc_t(grad)));
  }
  if constexpr (HAS_BUF) {
    // The new buffer stays in acc_t for the Nesterov term, as in torch.
    const acc_t buf =
        is_first_step
            ? acc_t(grad)
            : ::fma(acc_t(h.momentum), acc_t(momentum_buffer),
                    acc_t(1 - h.dampening) * acc_t(grad));
    momentum_buffer = static_cast<opmath_t>(buf);
    if constexpr (NESTEROV) {
      grad = static_cast<opmath_t>(::fma(acc_t(h.momentum), buf, acc_t(grad)));
    } else {
      grad = static_cast<opmath_t>(buf);
    }
  }
  param = static_cast<opmath_t>(::fma(-acc_t(h.lr), acc_t(grad), acc_t(param)));
}

// ---------------------------------------------------------------------------
// Adagrad. corrected_lr, weight_decay and eps are doubles, so the weight-decay
// term and the whole parameter update (including its divide) run in fp64;
// the state-sum accumulation stays in the math type.
// ---------------------------------------------------------------------------
struct AdagradHyper {
  double corrected_lr, weight_decay, eps;
};

// The first part of ATen's adagrad_math for one element: maximize, weight
// decay (into `grad`) and the state sum, whose square root the update takes.
template <typename opmath_t>
__device__ __forceinline__ void adagrad_sum(const opmath_t param, opmath_t& grad,
                                            opmath_t& state_sum, const AdagradHyper& h,
                                            const bool maximize) {
  if (maximize) {
    grad = -grad;
  }
  if (h.weight_decay != 0) {
    // grad += param * weight_decay
    grad = static_cast<opmath_t>(::fma(double(param), h.weight_decay, double(grad)));
  }
  // state_sum += grad * grad, in the math type
  state_sum = ::fma(grad, grad, state_sum);
}

// The rest, given `root` = sqrt(state_sum).
template <typename opmath_t>
__device__ __forceinline__ void adagrad_finish(opmath_t& param, const opmath_t grad,
                                               const opmath_t root, const AdagradHyper& h) {
  param = static_cast<opmath_t>(double(param) -
                                h.corrected_lr * double(grad) / (double(root) + h.eps));
}

template <typename opmath_t, bool ZEROS = false>
__device__ __forceinline__ void adagrad_element(
    opmath_t& param, opmath_t grad, opmath_t& state_sum, const AdagradHyper& h,
    const bool maximize) {
  adagrad_sum(param, grad, state_sum, h, maximize);
  adagrad_finish(param, grad, sqrt_rn<ZEROS>(state_sum), h);
}

// Float32 Adagrad (this build's explicitly non-ATen variant): the element loop
// of the reference's CPU kernel (src/torchstrap/kernels/csrc/cpu/adagrad.cpp:
// 94-156) -- every operation in float, the multiply-adds fused -- so on float32
// parameters it is bit-identical to the reference's CPU build, not to torch's
// fp64 device math.
struct AdagradF32Hyper {
  float corrected_lr, weight_decay, eps;
  bool has_weight_decay;
};

__device__ __forceinline__ void adagrad_sum_f32(const float param, float& grad, float& state_sum,
                                                const AdagradF32Hyper& h, const bool maximize) {
  if (maximize) {
    grad = -grad;
  }
  if (h.has_weight_decay) {
    grad = ::fmaf(param, h.weight_decay, grad);
  }
  state_sum = ::fmaf(grad, grad, state_sum);
}

// The rest, given `root` = sqrt(state_sum).
__device__ __forceinline__ void adagrad_finish_f32(float& param, const float grad, const float root,
                                                   const AdagradF32Hyper& h) {
  const float std_val = root + h.eps;
  param = param - (h.corrected_lr * grad) / std_val;
}

__device__ __forceinline__ void adagrad_element_f32(float& param, float grad, float& state_sum,
                                                    const AdagradF32Hyper& h,
                                                    const bool maximize) {
  adagrad_sum_f32(param, grad, state_sum, h, maximize);
  adagrad_finish_f32(param, grad, sqrt_rn(state_sum), h);
}

// The CPU kernel's corrected_lr: lr / (1 + (step - 1) * lr_decay) in double
// from the double step (cpu/adagrad.cpp:207-212), then narrowed to float.
__device__ __forceinline__ float adagrad_corrected_lr_f32(const double lr, const double lr_decay,
                                                          const double step) {
  return static_cast<float>(lr / ::fma(step - 1.0, lr_decay, 1.0));
}

// corrected_lr = lr / (1 + (step - 1) * lr_decay), with `step - 1` in float.
__device__ __forceinline__ double adagrad_corrected_lr(
    const double lr, const double lr_decay, const float step) {
  const double denom = ::fma(static_cast<double>(step - 1), lr_decay, 1.0);
  return lr / denom;
}

}  // namespace churten
