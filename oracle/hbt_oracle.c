/*
 * hbt_oracle.c - CPU restatement of the hot path's floating-point arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, the smoke() entry point and bench.py's
 * CPU-baseline leg load this oracle: to check results, or to time the reference's CPU
 * arithmetic.  The product (libhbt.so and the hybrid_training_amd package) never links
 * or calls it.
 *
 * Compiled with -ffp-contract=off so that only the fmaf() calls below fuse.
 *
 * Dtype codes: 0 float32, 1 bfloat16, 2 float16.  A 2-byte array holds the element's
 * bit pattern (uint16).  R_D(x) rounds an fp32 value to dtype D, to nearest even, and
 * widens it back exactly: the value a torch CPU op whose result has dtype D holds (it
 * computes in fp32 and rounds once).  R_float32 is the identity.
 *
 * What it restates:
 *   oracle_adamw - torch.optim.AdamW's single-tensor path on CPU tensors,
 *       torch/optim/adam.py:396-547 (torch 2.10.0), which the reference calls from
 *       optim/sharded_optimizer.py:111-120 and :355.  Per element, on tensors of dtype P
 *       (parameters, exp_avg, exp_avg_sq), each line one torch op rounded to P:
 *         param.mul_(1 - lr*wd)                    p * decay               (adam.py:416-419)
 *         exp_avg.lerp_(grad, 1 - beta1)           fma(w, g - m, m), |w| < 0.5
 *                                                  fma(w - 1, g - m, g) otherwise
 *                                                  (ATen's vectorised lerp, adam.py:457)
 *         exp_avg_sq.mul_(beta2)                   v * beta2               (adam.py:476)
 *           .addcmul_(grad, grad, value=1-beta2)   fma(c * g, g, v)        (contracted by the
 *                                                  AVX-512 build; pinned by the tests)
 *         denom = (exp_avg_sq.sqrt() / bc2_sqrt).add_(eps)                 (adam.py:545)
 *                                                  fp32: one expression; 2-byte P: sqrt, the
 *                                                  division and the add each rounded, and
 *                                                  eps itself rounded to P (torch rounds the
 *                                                  Python scalar of add_ to the tensor dtype)
 *         param.addcdiv_(exp_avg, denom, value=-step_size)  p + (s*m)/d    (adam.py:547)
 *       preceded by the unscale multiply (optim/grad_scaler.py:181-186) and the clip
 *       multiply (optim/sharded_optimizer.py:333-337) of the reference, each a
 *       grad.mul_ rounded to the gradient's dtype G.  For P = fp32 and G = bf16 (the
 *       loss-scaled configuration) the rounded bf16 gradient widens exactly into the fp32
 *       update; torch's AdamW itself refuses that pair, so that branch is this library's
 *       definition.  sqrt is correctly rounded (sqrtf) unless `sqrt_override` supplies
 *       the square roots to use; the tests pass torch's own exp_avg_sq.sqrt() there,
 *       which pins every other operation of the restatement bitwise against torch.
 *       `grad_out`, when non-null, receives the scaled gradient (the write-back).
 *   oracle_sgd - torch.optim.SGD's single-tensor path on CPU tensors,
 *       torch/optim/sgd.py (_single_tensor_sgd, torch 2.10.0), which the reference
 *       builds at optim/sharded_optimizer.py:121-126.  torch's CPU `add(.., alpha=a)`
 *       is one fused multiply-add with the alpha first rounded to the tensor dtype
 *       (pinned by the tests), `mul_` one rounded multiply by the fp32 scalar:
 *         grad = grad.add(param, alpha=wd)            fma(p, a(wd), g)      (wd != 0)
 *         buf = grad.clone()                           first step
 *         buf.mul_(m).add_(grad, alpha=1-dampening)    fma(g, a(1-d), buf*m) later steps
 *         grad = grad.add(buf, alpha=m) | buf          nesterov | plain
 *         param.add_(grad, alpha=-lr)                  fma(g, a(-lr), p)
 *       preceded by the unscale and clip multiplies, as for AdamW.  That is torch's
 *       vectorised body.  On 2-byte tensors torch's scalar remainder loop (the last
 *       n mod V elements of a tensor, V its vector width) rounds each alpha product to
 *       the dtype before the add instead; `remainder` selects that form (pinned by the
 *       tests) so the difference can be checked, while libhbt.so follows the body.
 *   oracle_sqnorm - sum of (double)(R_G(g * unscale))^2 with Neumaier compensation, the
 *       quantity NormContribution.squared_norm computes in fp64
 *       (optim/sharded_optimizer.py:145-158) over the unscaled gradient the in-place
 *       GradScaler.unscale_ stores.
 *   oracle_f32_to_bf16 - round-to-nearest-even narrowing with NaN -> 0x7FC0, the
 *       conversion behind Tensor.to(torch.bfloat16).
 *   oracle_adamw_f64, oracle_sgd_f64, oracle_sqnorm_f64 - the same three on float64
 *       tensors, whose every operation torch computes in double with the Python scalars
 *       unrounded (adam.py:396-547 and _single_tensor_sgd on float64; the reference's
 *       masters are float64 when the parameters are and mixed precision is off,
 *       parallel/fsdp.py:379-393): the op sequences above with every rounding the
 *       identity of double arithmetic, fma() where the fp32 restatement has fmaf(), the
 *       unscale and clip multiplies by the double factors, each square one rounded
 *       double product (g.to(float64).pow(2)).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float bits_to_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

static uint32_t f32_to_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    return u;
}

/* bf16: keep the high 16 bits, rounding the discarded low half to nearest, ties to the
 * even high half; NaN -> 0x7FC0. */
static uint16_t bf16_bits(float x) {
    if (isnan(x)) return 0x7FC0u;
    const uint32_t u = f32_to_bits(x);
    const uint32_t low = u & 0xFFFFu;
    uint32_t high = u >> 16;
    if (low > 0x8000u || (low == 0x8000u && (high & 1u))) high += 1u;
    return (uint16_t)high;
}

/* IEEE binary16 by its definition: a value below 2^-14 is a multiple of 2^-24; one in
 * [2^E, 2^(E+1)) a multiple of 2^(E-10).  Dividing by that quantum is an exact power-of-
 * two scaling and rintf() rounds to nearest even, so m * quantum is the correctly
 * rounded half.  Magnitudes that round past 65504 are infinite; NaN -> sign | 0x7E00. */
static uint16_t f16_bits(float x) {
    const uint16_t sign = (uint16_t)((f32_to_bits(x) >> 16) & 0x8000u);
    if (isnan(x)) return (uint16_t)(sign | 0x7E00u);
    const float a = fabsf(x);
    if (a >= 65520.0f) return (uint16_t)(sign | 0x7C00u);
    if (a < 6.103515625e-05f) { /* 2^-14: subnormal or zero (m == 1024 is the smallest normal) */
        const int m = (int)rintf(a * 16777216.0f);
        return (uint16_t)(sign | m);
    }
    int e = 0;
    (void)frexpf(a, &e); /* a in [2^(e-1), 2^e) */
    int exponent = e - 1;
    int m = (int)rintf(ldexpf(a, 10 - exponent)); /* in [1024, 2048] */
    if (m == 2048) {
        m = 1024;
        exponent += 1;
    }
    if (exponent > 15) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | ((exponent + 15) << 10) | (m - 1024));
}

static float f16_value(uint16_t h) {
    const float sign = (h & 0x8000u) ? -1.0f : 1.0f;
    const int exponent = (h >> 10) & 0x1F;
    const int mantissa = h & 0x3FF;
    if (exponent == 0) return sign * ldexpf((float)mantissa, -24);
    if (exponent == 31) return mantissa ? NAN : sign * INFINITY;
    return sign * ldexpf((float)(mantissa + 1024), exponent - 25);
}

static float round_to(float x, int dt) {
    if (dt == 1) return bits_to_f32((uint32_t)bf16_bits(x) << 16);
    if (dt == 2) return f16_value(f16_bits(x));
    return x;
}

static float load(const void* a, int64_t i, int dt) {
    if (dt == 0) return ((const float*)a)[i];
    const uint16_t h = ((const uint16_t*)a)[i];
    return dt == 1 ? bits_to_f32((uint32_t)h << 16) : f16_value(h);
}

/* x must already be representable in dt. */
static void store(void* a, int64_t i, float x, int dt) {
    if (dt == 0) {
        ((float*)a)[i] = x;
    } else {
        ((uint16_t*)a)[i] = dt == 1 ? bf16_bits(x) : f16_bits(x);
    }
}

void oracle_round(const float* x, float* out, int64_t n, int dt) {
    for (int64_t i = 0; i < n; ++i) out[i] = round_to(x[i], dt);
}

void oracle_adamw(void* p, const void* g, void* m, void* v, int64_t n, int pdt, int gdt, float unscale,
                  float grad_mul, float decay, float lerp_w, float beta2, float one_minus_beta2, float bc2_sqrt,
                  float eps, float neg_step, const float* sqrt_override, void* grad_out) {
    const int lerp_small = fabsf(lerp_w) < 0.5f;
    const float lerp_w_minus_1 = lerp_w - 1.0f;
    const float eps_p = round_to(eps, pdt);
    for (int64_t i = 0; i < n; ++i) {
        float gi = load(g, i, gdt);
        if (unscale != 1.0f) gi = round_to(gi * unscale, gdt);
        gi = round_to(gi * grad_mul, gdt);
        if (grad_out != 0) store(grad_out, i, gi, gdt);
        float pi = round_to(load(p, i, pdt) * decay, pdt);
        const float m0 = load(m, i, pdt);
        const float diff = gi - m0;
        const float mi = round_to(lerp_small ? fmaf(lerp_w, diff, m0) : fmaf(lerp_w_minus_1, diff, gi), pdt);
        float vi = round_to(load(v, i, pdt) * beta2, pdt);
        const float c = one_minus_beta2 * gi;
        vi = round_to(fmaf(c, gi, vi), pdt);
        const float root = sqrt_override != 0 ? sqrt_override[i] : sqrtf(vi);
        float denom;
        if (pdt == 0) {
            const float q = root / bc2_sqrt;
            denom = q + eps;
        } else {
            denom = round_to(round_to(round_to(root, pdt) / bc2_sqrt, pdt) + eps_p, pdt);
        }
        const float num = neg_step * mi;
        const float upd = num / denom;
        pi = round_to(pi + upd, pdt);
        store(p, i, pi, pdt);
        store(m, i, mi, pdt);
        store(v, i, vi, pdt);
    }
}

static void neumaier_add(double* sum, double* comp, double x) {
    const double t = *sum + x;
    if (fabs(*sum) >= fabs(x)) {
        *comp += (*sum - t) + x;
    } else {
        *comp += (x - t) + *sum;
    }
    *sum = t;
}

/* x + alpha * y as torch's CPU `add(.., alpha=)` on dtype dt: in its vectorised body one
 * fused multiply-add rounded once (for fp32 and, as the products of two 2-byte values
 * are exact in fp32, for 2-byte dtypes alike); in its scalar remainder loop on a 2-byte
 * dtype (`remainder` set) the product is first rounded to dt, as c10's 2-byte
 * arithmetic does. */
static float add_alpha(float x, float y, float alpha, int dt, int remainder) {
    if (remainder && dt != 0) return round_to(x + round_to(alpha * y, dt), dt);
    return round_to(fmaf(y, alpha, x), dt);
}

/* mode: 0 no momentum, 1 momentum first step (buf := g), 2 momentum.  `remainder`: the
 * arithmetic of torch's scalar remainder loop instead of its vectorised body (see
 * add_alpha; the two differ only there). */
void oracle_sgd(void* p, const void* g, void* buf, int64_t n, int pdt, int gdt, float unscale, float grad_mul,
                int apply_wd, float wd, int mode, float momentum, float one_minus_dampening, int nesterov,
                float neg_lr, void* grad_out, int remainder) {
    const float wd_a = round_to(wd, pdt);
    const float momentum_a = round_to(momentum, pdt);
    const float omd_a = round_to(one_minus_dampening, pdt);
    const float lr_a = round_to(neg_lr, pdt);
    for (int64_t i = 0; i < n; ++i) {
        float x = load(g, i, gdt);
        if (unscale != 1.0f) x = round_to(x * unscale, gdt);
        x = round_to(x * grad_mul, gdt);
        if (grad_out != 0) store(grad_out, i, x, gdt);
        const float pi = load(p, i, pdt);
        if (apply_wd) x = add_alpha(x, pi, wd_a, pdt, remainder);
        float b = 0.0f;
        if (mode == 1) {
            b = x;
        } else if (mode == 2) {
            b = round_to(load(buf, i, pdt) * momentum, pdt);
            b = add_alpha(b, x, omd_a, pdt, remainder);
        }
        if (mode != 0) {
            store(buf, i, b, pdt);
            x = nesterov ? add_alpha(x, b, momentum_a, pdt, remainder) : b;
        }
        store(p, i, add_alpha(pi, x, lr_a, pdt, remainder), pdt);
    }
}

double oracle_sqnorm(const void* g, int64_t n, int gdt, float unscale) {
    double sum = 0.0, comp = 0.0;
    for (int64_t i = 0; i < n; ++i) {
        float y = load(g, i, gdt);
        if (unscale != 1.0f) y = round_to(y * unscale, gdt);
        const double x = (double)y;
        neumaier_add(&sum, &comp, x * x);
    }
    return isfinite(sum) ? sum + comp : sum; /* an inf square keeps the sum inf */
}

void oracle_adamw_f64(double* p, const double* g, double* m, double* v, int64_t n, double unscale, double grad_mul,
                      double decay, double lerp_w, double beta2, double one_minus_beta2, double bc2_sqrt, double eps,
                      double neg_step, const double* sqrt_override, double* grad_out) {
    const int lerp_small = fabs(lerp_w) < 0.5;
    const double lerp_w_minus_1 = lerp_w - 1.0;
    for (int64_t i = 0; i < n; ++i) {
        double gi = g[i];
        if (unscale != 1.0) gi = gi * unscale;
        gi = gi * grad_mul;
        if (grad_out != 0) grad_out[i] = gi;
        const double pi = p[i] * decay;
        const double diff = gi - m[i];
        const double mi = lerp_small ? fma(lerp_w, diff, m[i]) : fma(lerp_w_minus_1, diff, gi);
        double vi = v[i] * beta2;
        vi = fma(one_minus_beta2 * gi, gi, vi);
        const double root = sqrt_override != 0 ? sqrt_override[i] : sqrt(vi);
        const double denom = root / bc2_sqrt + eps;
        p[i] = pi + (neg_step * mi) / denom;
        m[i] = mi;
        v[i] = vi;
    }
}

/* mode as for oracle_sgd; every alpha is the unrounded double. */
void oracle_sgd_f64(double* p, const double* g, double* buf, int64_t n, double unscale, double grad_mul,
                    int apply_wd, double wd, int mode, double momentum, double one_minus_dampening, int nesterov,
                    double neg_lr, double* grad_out) {
    for (int64_t i = 0; i < n; ++i) {
        double x = g[i];
        if (unscale != 1.0) x = x * unscale;
        x = x * grad_mul;
        if (grad_out != 0) grad_out[i] = x;
        const double pi = p[i];
        if (apply_wd) x = fma(pi, wd, x);
        if (mode == 1) {
            buf[i] = x;
        } else if (mode == 2) {
            buf[i] = fma(x, one_minus_dampening, buf[i] * momentum);
        }
        if (mode != 0) x = nesterov ? fma(buf[i], momentum, x) : buf[i];
        p[i] = fma(x, neg_lr, pi);
    }
}

double oracle_sqnorm_f64(const double* g, int64_t n) {
    double sum = 0.0, comp = 0.0;
    for (int64_t i = 0; i < n; ++i) neumaier_add(&sum, &comp, g[i] * g[i]);
    return isfinite(sum) ? sum + comp : sum;
}

void oracle_f32_to_bf16(const float* x, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = bf16_bits(x[i]);
}

void oracle_f32_to_f16(const float* x, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = f16_bits(x[i]);
}
