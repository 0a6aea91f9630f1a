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
 * What it restates:
 *   oracle_adamw_f32 - torch.optim.AdamW's single-tensor path on CPU tensors,
 *       torch/optim/adam.py:396-547 (torch 2.10.0), which the reference calls from
 *       optim/sharded_optimizer.py:111-120 and :355.  Per element, torch's CPU
 *       kernels compute:
 *         param.mul_(1 - lr*wd)                    p * decay               (adam.py:416-419)
 *         exp_avg.lerp_(grad, 1 - beta1)           fma(w, g - m, m), |w| < 0.5
 *                                                  fma(w - 1, g - m, g) otherwise
 *                                                  (ATen's vectorised lerp, adam.py:457)
 *         exp_avg_sq.mul_(beta2)                   v * beta2               (adam.py:476)
 *           .addcmul_(grad, grad, value=1-beta2)   fma(c * g, g, v)        (contracted by the
 *                                                  AVX-512 build; pinned by the tests)
 *         denom = (exp_avg_sq.sqrt() / bc2_sqrt).add_(eps)                 (adam.py:545)
 *         param.addcdiv_(exp_avg, denom, value=-step_size)  p + (s*m)/d    (adam.py:547)
 *       preceded by the unscale multiply (optim/grad_scaler.py:181-186) and the clip
 *       multiply (optim/sharded_optimizer.py:333-337) of the reference.
 *       sqrt is correctly rounded (sqrtf) unless `sqrt_override` supplies the square
 *       roots to use; the tests pass torch's own exp_avg_sq.sqrt() there, which pins
 *       every other operation of the restatement bitwise against torch.
 *   oracle_sgd - torch.optim.SGD's single-tensor path on CPU tensors,
 *       torch/optim/sgd.py (_single_tensor_sgd, torch 2.10.0), which the reference
 *       builds at optim/sharded_optimizer.py:121-126.  torch's CPU `add(.., alpha=a)`
 *       is one fused multiply-add (pinned by the tests), `mul_` one rounded multiply:
 *         grad = grad.add(param, alpha=wd)            fma(p, wd, g)      (wd != 0)
 *         buf = grad.clone()                           first step
 *         buf.mul_(m).add_(grad, alpha=1-dampening)    fma(g, 1-d, buf*m) later steps
 *         grad = grad.add(buf, alpha=m) | buf          nesterov | plain
 *         param.add_(grad, alpha=-lr)                  fma(g, -lr, p)
 *       preceded by the unscale and clip multiplies, as for AdamW.
 *   oracle_sqnorm_* - sum of (double)(g * unscale)^2 with Neumaier compensation, the
 *       quantity NormContribution.squared_norm computes in fp64
 *       (optim/sharded_optimizer.py:145-158).
 *   oracle_f32_to_bf16 - round-to-nearest-even narrowing with NaN -> 0x7FC0, the
 *       conversion behind Tensor.to(torch.bfloat16).
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

void oracle_adamw_f32(float* p, const float* g, float* m, float* v, int64_t n, float unscale,
                      float grad_mul, float decay, float lerp_w, float beta2,
                      float one_minus_beta2, float bc2_sqrt, float eps, float neg_step,
                      const float* sqrt_override) {
    const int lerp_small = fabsf(lerp_w) < 0.5f;
    const float lerp_w_minus_1 = lerp_w - 1.0f;
    for (int64_t i = 0; i < n; ++i) {
        float gi = g[i] * unscale;
        gi = gi * grad_mul;
        float pi = p[i] * decay;
        const float diff = gi - m[i];
        const float mi = lerp_small ? fmaf(lerp_w, diff, m[i]) : fmaf(lerp_w_minus_1, diff, gi);
        float vi = v[i] * beta2;
        const float c = one_minus_beta2 * gi;
        vi = fmaf(c, gi, vi);
        const float root = sqrt_override != 0 ? sqrt_override[i] : sqrtf(vi);
        const float q = root / bc2_sqrt;
        const float denom = q + eps;
        const float num = neg_step * mi;
        const float upd = num / denom;
        pi = pi + upd;
        p[i] = pi;
        m[i] = mi;
        v[i] = vi;
    }
}

/* The same update for bf16 gradients: each gradient is widened exactly to fp32. */
void oracle_adamw_bf16grad(float* p, const uint16_t* g, float* m, float* v, int64_t n,
                           float unscale, float grad_mul, float decay, float lerp_w, float beta2,
                           float one_minus_beta2, float bc2_sqrt, float eps, float neg_step) {
    for (int64_t i = 0; i < n; ++i) {
        const float gi = bits_to_f32((uint32_t)g[i] << 16);
        oracle_adamw_f32(p + i, &gi, m + i, v + i, 1, unscale, grad_mul, decay, lerp_w, beta2,
                         one_minus_beta2, bc2_sqrt, eps, neg_step, 0);
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

/* mode: 0 no momentum, 1 momentum first step (buf := g), 2 momentum. */
void oracle_sgd(float* p, const float* g, float* buf, int64_t n, float unscale, float grad_mul,
                int apply_wd, float wd, int mode, float momentum, float one_minus_dampening,
                int nesterov, float neg_lr) {
    for (int64_t i = 0; i < n; ++i) {
        float x = g[i];
        if (unscale != 1.0f) x = x * unscale;
        x = x * grad_mul;
        if (apply_wd) x = fmaf(p[i], wd, x);
        if (mode == 1) {
            buf[i] = x;
        } else if (mode == 2) {
            const float b = buf[i] * momentum;
            buf[i] = fmaf(x, one_minus_dampening, b);
        }
        if (mode != 0) x = nesterov ? fmaf(buf[i], momentum, x) : buf[i];
        p[i] = fmaf(x, neg_lr, p[i]);
    }
}

double oracle_sqnorm_f32(const float* g, int64_t n, float unscale) {
    double sum = 0.0, comp = 0.0;
    for (int64_t i = 0; i < n; ++i) {
        const double x = (double)(g[i] * unscale);
        neumaier_add(&sum, &comp, x * x);
    }
    return isfinite(sum) ? sum + comp : sum; /* an inf square keeps the sum inf */
}

double oracle_sqnorm_bf16(const uint16_t* g, int64_t n, float unscale) {
    double sum = 0.0, comp = 0.0;
    for (int64_t i = 0; i < n; ++i) {
        const double x = (double)(bits_to_f32((uint32_t)g[i] << 16) * unscale);
        neumaier_add(&sum, &comp, x * x);
    }
    return isfinite(sum) ? sum + comp : sum;
}

void oracle_f32_to_bf16(const float* x, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        if (isnan(x[i])) {
            out[i] = 0x7FC0u;
            continue;
        }
        /* Keep the high 16 bits, rounding the discarded low half to nearest, ties to
         * the even high half. */
        const uint32_t u = f32_to_bits(x[i]);
        const uint32_t low = u & 0xFFFFu;
        uint32_t high = u >> 16;
        if (low > 0x8000u || (low == 0x8000u && (high & 1u))) high += 1u;
        out[i] = (uint16_t)high;
    }
}
