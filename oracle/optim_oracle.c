/*
 * optim_oracle.c -- TEST INFRASTRUCTURE ONLY. CPU restatement of the
 * reference's fused batched optimizer step, used as the checker for the HIP
 * kernels. Nothing in churten_amd/ may load or call this file; only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg do.
 *
 * Two formulations of each optimizer, because the reference itself has two
 * (each bit-identical to torch's fused kernel on its own device):
 *
 *   ORACLE_DEVICE  the element math the reference's GPU kernels run: ATen's
 *                  device `adam_math` / `adagrad_math` (called verbatim at
 *                  src/torchstrap/kernels/csrc/cuda/adam.cu:146-157 and
 *                  cuda/adagrad.cu:141-148) and `sgd_math` (transcribed at
 *                  cuda/sgd.cu:90-132), in the form torch 2.10.0+rocm7.0 ships
 *                  for ROCm (ATen/native/hip/fused_adam_utils.cuh:28-92,
 *                  131-139; fused_adagrad_utils.cuh:16-50, 75-81; SGD's ROCm
 *                  source is not shipped -- its form, double hyperparameters,
 *                  is pinned by torch._fused_sgd_ on the MI355X). The HIP
 *                  kernels must match this bit for bit.
 *   ORACLE_CPU     the reference's own CPU kernels: per-replica double prologue,
 *                  AVX2 vector body of 8 lanes plus a scalar tail at the end of
 *                  each row (cpu/adam.cpp:152-322, cpu/sgd.cpp:110-283,
 *                  cpu/adagrad.cpp:94-233, chunking cpu/consolidated.h:26-51).
 *                  The HIP kernels must agree with it to atol = rtol = 1e-5.
 *
 * Every multiply-add that the reference's compiler contracts is written as an
 * explicit fma() here and the file is compiled with -ffp-contract=off, so the
 * rounding sequence is fixed by this source alone. Division and sqrt are IEEE
 * correctly rounded on both sides.
 *
 * Parity pinning (what checks this file, tests/test_oracle_*.py):
 *   ORACLE_CPU    bit-exact against golden vectors written by the reference's
 *                 CPU kernels compiled from /root/reference (oracle/Makefile,
 *                 tests/golden/make_cpu_golden.py), and live against that build
 *                 when it is present; closed forms (first Adam step from zero
 *                 moments, momentum-0 SGD, first Adagrad step, frozen rows).
 *   ORACLE_DEVICE bit-exact against golden vectors written by torch's ROCm
 *                 fused kernels on the MI355X (tests/golden/make_device_golden.py);
 *                 the same closed forms.
 *
 * Layout: contiguous row-major (R, T) float32 arrays; `steps` is (R,) float32
 * and is bumped in place (steps[r] += mask[r]) before the update, as every
 * reference operator does (cuda/adam.cu:277, cpu/adam.cpp:341).
 *
 * bfloat16 optimizer state (this build's extension; the reference operators
 * reject mixed dtypes): the state is held here as float32 arrays of
 * bfloat16-representable values; the step is the float32 step above, after
 * which oracle_round_bf16_rows rounds the active rows' state to nearest-even
 * bfloat16. Pinned against torch's own float -> bfloat16 conversion
 * (tests/test_oracle_bf16_state.py).
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#define ORACLE_DEVICE 0
#define ORACLE_CPU 1

/* Vector width of the reference CPU build: AVX2 (setup.py:60), 8 floats. */
#define CPU_LANES 8
/* Elements per CPU task (cpu/consolidated.h:26); a multiple of CPU_LANES, so
 * the scalar tail only ever falls at the end of a row. */
#define CPU_CHUNK 16384

static void bump(float* steps, const uint8_t* mask, int64_t R) {
  for (int64_t r = 0; r < R; ++r) {
    steps[r] = steps[r] + (mask[r] ? 1.0f : 0.0f);
  }
}

/* x86 maxps semantics as ATen's AVX2 `maximum` uses them
 * (a > b ? a : b, with any NaN operand giving an all-ones NaN). */
static float vec_maximum(float a, float b) {
  if (isnan(a) || isnan(b)) {
    union { uint32_t u; float f; } nan_bits = {0xFFFFFFFFu};
    return nan_bits.f;
  }
  return a > b ? a : b;
}

/* std::max(a, b): b if a < b, else a. */
static float std_max(float a, float b) { return a < b ? b : a; }

/* ======================================================================== */
/* Adam / AdamW                                                             */
/* ======================================================================== */

/* ATen device adam_math (fused_adam_utils.cuh:28-92) on one element, with
 * hyperparameters in double and the bias corrections already narrowed. */
static void adam_device_elem(float* p, float g, float* m, float* v, float* mx,
                             double lr, double b1, double b2, double wd,
                             double eps, int amsgrad, int adamw, int maximize,
                             float bc1, float bc2s) {
  float param = *p;
  float grad = g;
  if (maximize) grad = -grad;
  if (wd != 0) {
    if (adamw) {
      /* param -= lr * wd * param, in double */
      param = (float)fma(-(lr * wd), (double)param, (double)param);
    } else {
      /* grad += param * wd, in double */
      grad = (float)fma((double)param, wd, (double)grad);
    }
  }
  /* exp_avg = beta1 * exp_avg + (1 - beta1) * grad, in double */
  const float exp_avg = (float)fma(b1, (double)*m, (1 - b1) * (double)grad);
  /* exp_avg_sq = beta2 * exp_avg_sq + (1 - beta2) * grad * grad */
  const float exp_avg_sq =
      (float)fma(b2, (double)*v, ((1 - b2) * (double)grad) * (double)grad);
  const float step_size = (float)(lr / (double)bc1);
  float denom;
  if (amsgrad) {
    const float mxv = fmaxf(*mx, exp_avg_sq);
    *mx = mxv;
    denom = (float)((double)(sqrtf(mxv) / bc2s) + eps);
  } else {
    denom = (float)((double)(sqrtf(exp_avg_sq) / bc2s) + eps);
  }
  param = param - (step_size * exp_avg) / denom;
  *p = param;
  *m = exp_avg;
  *v = exp_avg_sq;
}

typedef struct {
  float step_size, beta2, exp_avg_coeff, exp_avg_sq_coeff, bc2s, eps, wd, wd_mul;
  int has_wd, lerp_small;
} adam_cpu_consts;

/* Per-replica double prologue of the reference CPU kernel
 * (cpu/adam.cpp:333-358), narrowed where it narrows. */
static adam_cpu_consts adam_cpu_prologue(float lr, float b1, float b2,
                                         float eps, float wd, float step) {
  const double lr_d = lr, b1_d = b1, b2_d = b2, eps_d = eps, wd_d = wd;
  const double step_d = step;
  const double bc1 = 1 - pow(b1_d, step_d);
  const double bc2 = 1 - pow(b2_d, step_d);
  adam_cpu_consts c;
  c.step_size = (float)(lr_d / bc1);
  c.beta2 = (float)b2_d;
  c.exp_avg_coeff = (float)(1 - b1_d);
  c.exp_avg_sq_coeff = (float)(1 - b2_d);
  c.bc2s = (float)sqrt(bc2);
  c.eps = (float)eps_d;
  c.wd = (float)wd_d;
  c.wd_mul = (float)fma(-lr_d, wd_d, 1.0); /* 1 - lr * wd, contracted */
  c.has_wd = wd_d != 0.0;
  c.lerp_small = fabsf(c.exp_avg_coeff) < 0.5f;
  return c;
}

/* Vector-body element (cpu/adam.cpp:226-263). */
static void adam_cpu_vec_elem(float* p, float g, float* m, float* v, float* mx,
                              const adam_cpu_consts* c, int amsgrad, int adamw,
                              int maximize) {
  float param = *p;
  float grad = g;
  if (maximize) grad = grad * -1.0f;
  if (c->has_wd) {
    if (adamw) param = param * c->wd_mul;
    else grad = fmaf(param, c->wd, grad);
  }
  const float coeff = c->lerp_small ? c->exp_avg_coeff : c->exp_avg_coeff - 1.0f;
  const float base = c->lerp_small ? *m : grad;
  const float exp_avg = fmaf(coeff, grad - *m, base);
  /* Loadu(v) * beta2 + coeff * grad * grad: the compiler fuses the second
   * product into the add. */
  const float exp_avg_sq = fmaf(c->exp_avg_sq_coeff * grad, grad, *v * c->beta2);
  float denom;
  if (amsgrad) {
    const float mxv = vec_maximum(*mx, exp_avg_sq);
    *mx = mxv;
    denom = sqrtf(mxv) / c->bc2s + c->eps;
  } else {
    denom = sqrtf(exp_avg_sq) / c->bc2s + c->eps;
  }
  param = param + ((-c->step_size) * exp_avg) / denom;
  *p = param;
  *m = exp_avg;
  *v = exp_avg_sq;
}

/* Scalar element: the row tail and the strided path (cpu/adam.cpp:152-202). */
static void adam_cpu_scalar_elem(float* p, float g, float* m, float* v,
                                 float* mx, const adam_cpu_consts* c,
                                 int amsgrad, int adamw, int maximize) {
  float param = *p;
  float grad = g;
  if (maximize) grad = -grad;
  if (c->has_wd) {
    if (adamw) param = param * c->wd_mul;
    else grad = fmaf(param, c->wd, grad);
  }
  float exp_avg = *m;
  if (c->lerp_small) {
    exp_avg = fmaf(c->exp_avg_coeff, grad - exp_avg, exp_avg);
  } else {
    exp_avg = fmaf(-(grad - exp_avg), 1.0f - c->exp_avg_coeff, grad);
  }
  /* v = v * beta2; v = v + coeff * grad * grad: here the first product is
   * the one fused into the add. */
  const float exp_avg_sq = fmaf(*v, c->beta2, (c->exp_avg_sq_coeff * grad) * grad);
  float denom;
  if (amsgrad) {
    const float mxv = std_max(*mx, exp_avg_sq);
    *mx = mxv;
    denom = sqrtf(mxv) / c->bc2s + c->eps;
  } else {
    denom = sqrtf(exp_avg_sq) / c->bc2s + c->eps;
  }
  param = param - (c->step_size * exp_avg) / denom;
  *p = param;
  *m = exp_avg;
  *v = exp_avg_sq;
}

int oracle_adam_step(int form, float* p, const float* g, float* m, float* v,
                     float* mx, float* steps, const float* lr, const float* b1,
                     const float* b2, const float* eps, const float* wd,
                     const uint8_t* mask, int64_t R, int64_t T, int amsgrad,
                     int adamw, int maximize, int unit_stride) {
  bump(steps, mask, R);
  for (int64_t r = 0; r < R; ++r) {
    if (!mask[r]) continue;
    float* pr = p + r * T;
    const float* gr = g + r * T;
    float* mr = m + r * T;
    float* vr = v + r * T;
    float* xr = amsgrad ? mx + r * T : NULL;
    if (form == ORACLE_DEVICE) {
      const double bc1 = 1 - pow((double)b1[r], (double)steps[r]);
      const double bc2 = 1 - pow((double)b2[r], (double)steps[r]);
      const float bc1f = (float)bc1, bc2sf = (float)sqrt(bc2);
      for (int64_t t = 0; t < T; ++t) {
        adam_device_elem(pr + t, gr[t], mr + t, vr + t, xr ? xr + t : NULL,
                         lr[r], b1[r], b2[r], wd[r], eps[r], amsgrad, adamw,
                         maximize, bc1f, bc2sf);
      }
    } else {
      const adam_cpu_consts c =
          adam_cpu_prologue(lr[r], b1[r], b2[r], eps[r], wd[r], steps[r]);
      const int64_t vec_end = unit_stride ? T - (T % CPU_LANES) : 0;
      for (int64_t t = 0; t < T; ++t) {
        if (t < vec_end)
          adam_cpu_vec_elem(pr + t, gr[t], mr + t, vr + t, xr ? xr + t : NULL,
                            &c, amsgrad, adamw, maximize);
        else
          adam_cpu_scalar_elem(pr + t, gr[t], mr + t, vr + t,
                               xr ? xr + t : NULL, &c, amsgrad, adamw, maximize);
      }
    }
  }
  return 0;
}

/* ======================================================================== */
/* SGD                                                                      */
/* ======================================================================== */

/* Device sgd_math with double hyperparameters (form of cuda/sgd.cu:90-132 as
 * torch's ROCm build instantiates it). */
static void sgd_device_elem(float* p, float g, float* mb, double lr, double mom,
                            double damp, double wd, int has_buf, int nesterov,
                            int maximize, int first) {
  float param = *p;
  float grad = g;
  if (maximize) grad = (float)((double)grad * -1.0);
  if (wd != 0) grad = (float)fma(wd, (double)param, (double)grad);
  if (has_buf) {
    const double buf = first ? (double)grad
                             : fma(mom, (double)*mb, (1 - damp) * (double)grad);
    *mb = (float)buf;
    if (nesterov) grad = (float)fma(mom, buf, (double)grad);
    else grad = (float)buf;
  }
  *p = (float)fma(-lr, (double)grad, (double)param);
}

typedef struct {
  float wd, mom, one_minus_damp, lr, neg_lr;
  int has_wd, first;
} sgd_cpu_consts;

/* cpu/sgd.cpp:106-142 (scalar) and 148-193 (vector body). */
static void sgd_cpu_elem(float* p, float g, float* mb, const sgd_cpu_consts* c,
                         int has_buf, int nesterov, int maximize, int vec) {
  float param = *p;
  float grad = g;
  if (maximize) grad = vec ? grad * -1.0f : -grad;
  if (c->has_wd) grad = fmaf(param, c->wd, grad);
  if (has_buf) {
    float buf;
    if (c->first) buf = grad;
    else if (vec) buf = fmaf(c->one_minus_damp, grad, *mb * c->mom);
    else buf = fmaf(*mb, c->mom, grad * c->one_minus_damp);
    *mb = buf;
    if (nesterov) grad = fmaf(buf, c->mom, grad);
    else grad = buf;
  }
  *p = vec ? fmaf(grad, c->neg_lr, param) : fmaf(-grad, c->lr, param);
}

int oracle_sgd_step(int form, float* p, const float* g, float* mb,
                    float* steps, const float* lr, const float* mom,
                    const float* damp, const float* wd, const uint8_t* mask,
                    int64_t R, int64_t T, int nesterov, int maximize,
                    int unit_stride) {
  const int has_buf = mb != NULL;
  if (nesterov && !has_buf) return 1;
  bump(steps, mask, R);
  for (int64_t r = 0; r < R; ++r) {
    if (!mask[r]) continue;
    float* pr = p + r * T;
    const float* gr = g + r * T;
    float* br = has_buf ? mb + r * T : NULL;
    if (form == ORACLE_DEVICE) {
      const int first = steps[r] == 1.0f;
      for (int64_t t = 0; t < T; ++t)
        sgd_device_elem(pr + t, gr[t], br ? br + t : NULL, lr[r], mom[r],
                        damp[r], wd[r], has_buf, nesterov, maximize, first);
    } else {
      sgd_cpu_consts c;
      c.wd = wd[r];
      c.mom = mom[r];
      c.one_minus_damp = (float)(1 - (double)damp[r]);
      c.lr = lr[r];
      c.neg_lr = (float)(-(double)lr[r]);
      c.has_wd = (double)wd[r] != 0.0;
      c.first = (double)steps[r] == 1.0;
      const int64_t vec_end = unit_stride ? T - (T % CPU_LANES) : 0;
      for (int64_t t = 0; t < T; ++t)
        sgd_cpu_elem(pr + t, gr[t], br ? br + t : NULL, &c, has_buf, nesterov,
                     maximize, t < vec_end);
    }
  }
  return 0;
}

/* ======================================================================== */
/* Adagrad                                                                  */
/* ======================================================================== */

/* Device adagrad_math (fused_adagrad_utils.cuh:16-50): fp64 update. */
static void adagrad_device_elem(float* p, float g, float* s, double clr,
                                double wd, double eps, int maximize) {
  float param = *p;
  float grad = g;
  if (maximize) grad = -grad;
  if (wd != 0) grad = (float)fma((double)param, wd, (double)grad);
  const float sum = fmaf(grad, grad, *s);
  *s = sum;
  *p = (float)((double)param - (clr * (double)grad) / ((double)sqrtf(sum) + eps));
}

/* cpu/adagrad.cpp:94-156: float element loop (vector body and tail agree). */
static void adagrad_cpu_elem(float* p, float g, float* s, float clr, float wd,
                             float eps, int has_wd, int maximize, int vec) {
  float param = *p;
  float grad = g;
  if (maximize) grad = vec ? grad * -1.0f : -grad;
  if (has_wd) grad = fmaf(param, wd, grad);
  const float sum = fmaf(grad, grad, *s);
  *s = sum;
  const float std_val = sqrtf(sum) + eps;
  *p = param - (clr * grad) / std_val;
}

int oracle_adagrad_step(int form, float* p, const float* g, float* s,
                        float* steps, const float* lr, const float* lr_decay,
                        const float* wd, const float* eps, const uint8_t* mask,
                        int64_t R, int64_t T, int maximize, int unit_stride) {
  bump(steps, mask, R);
  for (int64_t r = 0; r < R; ++r) {
    if (!mask[r]) continue;
    float* pr = p + r * T;
    const float* gr = g + r * T;
    float* sr = s + r * T;
    if (form == ORACLE_DEVICE) {
      /* corrected_lr = lr / (1 + (step - 1) * lr_decay), step - 1 in float
       * (fused_adagrad_utils.cuh:75-81) */
      const double denom = fma((double)(steps[r] - 1.0f), (double)lr_decay[r], 1.0);
      const double clr = (double)lr[r] / denom;
      for (int64_t t = 0; t < T; ++t)
        adagrad_device_elem(pr + t, gr[t], sr + t, clr, wd[r], eps[r], maximize);
    } else {
      /* cpu/adagrad.cpp:207-218 */
      const double step = steps[r];
      const double clr = (double)lr[r] / fma(step - 1.0, (double)lr_decay[r], 1.0);
      const int64_t vec_end = unit_stride ? T - (T % CPU_LANES) : 0;
      for (int64_t t = 0; t < T; ++t)
        adagrad_cpu_elem(pr + t, gr[t], sr + t, (float)clr, wd[r], eps[r],
                         (double)wd[r] != 0.0, maximize, t < vec_end);
    }
  }
  return 0;
}

/* ======================================================================== */
/* bfloat16 state                                                           */
/* ======================================================================== */

/* float32 -> bfloat16 -> float32, round to nearest even; NaN -> 0x7FC0. */
static float round_bf16(float x) {
  uint32_t u;
  memcpy(&u, &x, sizeof u);
  if ((u & 0x7fffffffu) > 0x7f800000u) {
    u = 0x7fc00000u;
  } else {
    u += 0x7fffu + ((u >> 16) & 1u);
    u &= 0xffff0000u;
  }
  memcpy(&x, &u, sizeof x);
  return x;
}

/* Rounds rows r with mask[r] != 0 of the (R, T) array x to bfloat16 in place. */
int oracle_round_bf16_rows(float* x, const uint8_t* mask, int64_t R, int64_t T) {
  for (int64_t r = 0; r < R; ++r) {
    if (!mask[r]) continue;
    for (int64_t t = 0; t < T; ++t) x[r * T + t] = round_bf16(x[r * T + t]);
  }
  return 0;
}

int oracle_version(void) { return 2; }
