// Fused clip + AdamW / SGD steps, the deterministic fp64 gradient norm, the FSDP
// gradient local share, in-place gradient scaling and no_sync accumulation (gfx950).
//
// Every kernel streams its operands exactly once from HBM with 8- or 16-byte
// non-temporal vector loads and stores.  Work is split into fixed-size tiles; a launch
// covers a table of up to HBT_MAX_TENSORS_PER_LAUNCH tensors, so a list of flat shards
// (or of DDP-style per-parameter tensors) costs one launch per 16 tensors.
//
// Dtypes are template parameters given as HBT_DTYPE_* codes.  Arithmetic runs in fp32
// and, wherever a tensor of a 2-byte dtype holds an intermediate result, is rounded to
// that dtype (round_to<D>), as torch's CPU ops on bf16 / fp16 tensors compute in fp32 and
// round each result once.  For fp32 every rounding is the identity.
#include <cmath>
#include <cstring>
#include <mutex>

#include "hbt_common.hpp"

// Static scratch of hbt_grad_norm_noalloc: its per-chunk norm partials live here rather
// than in a caller or library allocation.  Every device holds its own copy (2 MiB) until
// the process ends.  In host code `scratch` names a host-side stand-in, not device memory:
// the device address is looked up once per device with hipGetSymbolAddress
// (noalloc_scratch below) and only that address is passed to kernels.
static __device__ __align__(256) double scratch[HBT_NOALLOC_MAX_PARTIALS];

namespace hbt {
namespace {

constexpr int kMaxT = HBT_MAX_TENSORS_PER_LAUNCH;
constexpr int F32 = HBT_DTYPE_F32;
constexpr int BF16 = HBT_DTYPE_BF16;
constexpr int F16 = HBT_DTYPE_F16;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int D>
constexpr int64_t bytes_of() { return D == F32 ? 4 : (D == HBT_DTYPE_F64 ? 8 : 2); }

template <int RD>
__device__ __forceinline__ u32x4 pack8_rounded(const float (&y)[8]) {
    uint32_t o[4];
    pack_rounded<RD, 4>(y, o);
    return u32x4{o[0], o[1], o[2], o[3]};
}

// ---- vector memory helpers ----------------------------------------------------------
// Every operand is touched exactly once per step, so loads and stores are marked
// non-temporal: the lines are not kept in L2/MALL for reuse that never comes.
//
// K consecutive elements of dtype D starting at element e of `base`, widened exactly to
// fp32, with one vector load of K * bytes(D) bytes (16 for 4 fp32 or 8 bf16/fp16, 8 for
// 4 bf16/fp16).
template <int D, int K>
__device__ __forceinline__ void load_vec(const void* base, int64_t e, float (&x)[K]) {
    static_assert(D == F32 || D == BF16 || D == F16, "vector loads move fp32, bf16 and fp16");
    if constexpr (D == F32) {
        static_assert(K == 4, "fp32 vectors are four elements");
        const f32x4 w = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(static_cast<const float*>(base) + e));
        x[0] = w.x;
        x[1] = w.y;
        x[2] = w.z;
        x[3] = w.w;
    } else if constexpr (K == 4) {
        const u32x2 w = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(base) + e));
        x[0] = b16_to_f32<D == F16>(w.x & 0xFFFFu);
        x[1] = b16_to_f32<D == F16>(w.x >> 16);
        x[2] = b16_to_f32<D == F16>(w.y & 0xFFFFu);
        x[3] = b16_to_f32<D == F16>(w.y >> 16);
    } else {
        static_assert(K == 8, "2-byte vectors are four or eight elements");
        const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(base) + e));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[2 * i] = b16_to_f32<D == F16>(w[i] & 0xFFFFu);
            x[2 * i + 1] = b16_to_f32<D == F16>(w[i] >> 16);
        }
    }
}
// Stores K values, each already representable in D (so the narrowing is exact).
template <int D, int K>
__device__ __forceinline__ void store_vec(void* base, int64_t e, const float (&x)[K]) {
    static_assert(D == F32 || D == BF16 || D == F16, "vector stores move fp32, bf16 and fp16");
    if constexpr (D == F32) {
        static_assert(K == 4, "fp32 vectors are four elements");
        __builtin_nontemporal_store(f32x4{x[0], x[1], x[2], x[3]}, reinterpret_cast<f32x4*>(static_cast<float*>(base) + e));
    } else if constexpr (K == 4) {
        uint32_t w[2];
        pack_rounded<D, 2>(x, w);
        __builtin_nontemporal_store(u32x2{w[0], w[1]}, reinterpret_cast<u32x2*>(static_cast<uint16_t*>(base) + e));
    } else {
        static_assert(K == 8, "2-byte vectors are four or eight elements");
        __builtin_nontemporal_store(pack8_rounded<D>(x), reinterpret_cast<u32x4*>(static_cast<uint16_t*>(base) + e));
    }
}
template <int D>
__device__ __forceinline__ float load_one(const void* base, int64_t e) {
    if constexpr (D == F32) return static_cast<const float*>(base)[e];
    return b16_to_f32<D == F16>(static_cast<const uint16_t*>(base)[e]);
}
template <int D>
__device__ __forceinline__ void store_one(void* base, int64_t e, float x) {
    if constexpr (D == F32) {
        static_cast<float*>(base)[e] = x;
    } else {
        static_cast<uint16_t*>(base)[e] = static_cast<uint16_t>(f32_to_b16<D == F16>(x));
    }
}

// K consecutive doubles from element e (K even, e a multiple of 2, base 16-byte aligned):
// K / 2 non-temporal 16-byte loads.
typedef double f64x2 __attribute__((ext_vector_type(2)));
template <int K>
__device__ __forceinline__ void load_f64(const void* base, int64_t e, double (&x)[K]) {
    static_assert(K % 2 == 0, "double vectors are two elements");
    const f64x2* p = reinterpret_cast<const f64x2*>(static_cast<const double*>(base) + e);
#pragma unroll
    for (int i = 0; i < K / 2; ++i) {
        const f64x2 w = __builtin_nontemporal_load(p + i);
        x[2 * i] = w.x;
        x[2 * i + 1] = w.y;
    }
}
template <int K>
__device__ __forceinline__ void store_f64(void* base, int64_t e, const double (&x)[K]) {
    static_assert(K % 2 == 0, "double vectors are two elements");
    f64x2* p = reinterpret_cast<f64x2*>(static_cast<double*>(base) + e);
#pragma unroll
    for (int i = 0; i < K / 2; ++i) __builtin_nontemporal_store(f64x2{x[2 * i], x[2 * i + 1]}, p + i);
}
// Four consecutive SB-byte elements (float64, float32, or bf16 / fp16 when SH) from
// element e, widened exactly to double (Tensor.to(float64)), with 16-byte loads (8-byte
// for 2-byte elements); base + e * SB must be aligned to 4 * SB bytes (16 for doubles).
template <int SB, bool SH>
__device__ __forceinline__ void load4_as_f64(const void* base, int64_t e, double (&x)[4]) {
    if constexpr (SB == 8) {
        load_f64<4>(base, e, x);
    } else {
        float f[4];
        load_vec<dtype_of<SB, SH>(), 4>(base, e, f);
#pragma unroll
        for (int c = 0; c < 4; ++c) x[c] = static_cast<double>(f[c]);
    }
}

// Wait for every outstanding vector-memory load of this wave (s_waitcnt vmcnt(0)).
// Issuing a lane's operand streams one after the other, rather than all at once, keeps
// the HBM request mix per wave simpler, and streamed faster.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// The table entry owning workgroup `block`: the last t with first[t] <= block.
__device__ __forceinline__ int owning_tensor(const int64_t* first, int32_t count, int64_t block) {
    int t = 0;
    while (t + 1 < count && block >= first[t + 1]) ++t;
    return t;
}

// The gradient after the reference's in-place multiplies: the unscale (GradScaler.unscale_,
// skipped when the factor is 1) and the clip, each computed in fp32 and rounded to the
// gradient's dtype GD, as grad.mul_(python float) on a GD tensor does.
template <int GD, bool kUnscale>
__device__ __forceinline__ float scaled_grad(float g, float unscale, float gmul) {
    if constexpr (kUnscale) g = round_to<GD>(g * unscale);
    return round_to<GD>(g * gmul);
}

// ---- AdamW -----------------------------------------------------------------------
// 32-thread workgroups, i.e. half a wavefront each, two 16-byte vectors per lane and
// fp32 operand: 256 elements per workgroup (512 for 2-byte parameters, whose 16-byte
// vectors hold eight).  Of the workgroup sizes, vector counts and persistent variants
// tried on the fp32 4-read / 3-write stream, this short-lived shape streamed fastest.
constexpr int kAdamBlock = 32;
// Vectors per lane: two for the step alone; one when the scaled gradient is also written
// back (4 reads and 4 writes per element), which was faster there; without the
// write-back the two tie.
template <bool kWriteBack>
constexpr int adam_unroll() { return kWriteBack ? 1 : 2; }
template <int PD>
constexpr int adam_vec() { return PD == F32 ? 4 : 8; }
template <int PD, bool kWriteBack>
constexpr int64_t adam_tile() { return int64_t(kAdamBlock) * adam_vec<PD>() * adam_unroll<kWriteBack>(); }
// Elements per workgroup of the AdamW and SGD kernels for a parameter dtype.
inline int64_t adam_tile_of(int32_t param_dtype, bool write_back) {
    if (param_dtype == F32) return write_back ? adam_tile<F32, true>() : adam_tile<F32, false>();
    return write_back ? adam_tile<BF16, true>() : adam_tile<BF16, false>();
}
// The AdamW kernel's shape: the one above for fp32 masters, whose update is bound by HBM.
// For 2-byte masters the rounding after every op makes the update VALU-bound, and a
// half-wave workgroup leaves half of every VALU instruction idle: full 64-lane waves with
// one vector per lane (512 elements, 1 KB per stream per workgroup; 46 VGPRs for bf16).
template <int PD>
constexpr int adamw_block() { return PD == F32 ? kAdamBlock : 64; }
template <int PD, bool kWriteBack>
constexpr int adamw_unroll() { return PD == F32 ? adam_unroll<kWriteBack>() : 1; }
template <int PD, bool kWriteBack>
constexpr int64_t adamw_tile() { return int64_t(adamw_block<PD>()) * adam_vec<PD>() * adamw_unroll<PD, kWriteBack>(); }
inline int64_t adamw_tile_of(int32_t param_dtype, bool write_back) {
    if (param_dtype == F32) return write_back ? adamw_tile<F32, true>() : adamw_tile<F32, false>();
    return write_back ? adamw_tile<BF16, true>() : adamw_tile<BF16, false>();
}
inline int adamw_block_of(int32_t param_dtype) { return param_dtype == F32 ? adamw_block<F32>() : adamw_block<BF16>(); }

struct AdamTable {
    void* p[kMaxT];
    void* g[kMaxT];
    void* m[kMaxT];
    void* v[kMaxT];
    int64_t n[kMaxT];
    int64_t first_block[kMaxT + 1];
    int32_t vec_ok[kMaxT];
    int32_t count;
};

struct AdamScalars {
    float unscale;
    float decay;
    float lerp_w;
    float lerp_w_minus_1;
    float beta2;
    float one_minus_beta2;
    float bc2_sqrt;
    float eps;  // rounded to the parameter dtype (torch's add_ of a Python scalar rounds it)
    float neg_step;
};

// One element of torch's single-tensor AdamW on tensors of dtype PD, given the already
// scaled gradient g.  Compiled with -ffp-contract=off: only the two explicit fmaf calls
// fuse.  For PD = fp32 this is exactly
//   p *= decay; m = lerp(m, g, w); v = v * beta2 + (1 - beta2) g^2;
//   p += (neg_step * m) / (sqrt(v) / bc2_sqrt + eps)
// and for a 2-byte PD each op of that sequence that torch runs as its own tensor op
// (mul_, lerp_, mul_, addcmul_, sqrt, div, add_, addcdiv_) rounds its result to PD.
template <int PD, bool kLerpSmall>
__device__ __forceinline__ void adamw_update(float& p, float g, float& m, float& v, const AdamScalars& s) {
    p = round_to<PD>(p * s.decay);
    const float diff = g - m;
    if constexpr (kLerpSmall) {
        m = round_to<PD>(__builtin_fmaf(s.lerp_w, diff, m));
    } else {
        m = round_to<PD>(__builtin_fmaf(s.lerp_w_minus_1, diff, g));
    }
    v = round_to<PD>(v * s.beta2);
    v = round_to<PD>(__builtin_fmaf(s.one_minus_beta2 * g, g, v));
    float denom;
    if constexpr (PD == F32) {
        denom = __builtin_sqrtf(v) / s.bc2_sqrt + s.eps;
    } else {
        denom = round_to<PD>(round_to<PD>(round_to<PD>(__builtin_sqrtf(v)) / s.bc2_sqrt) + s.eps);
    }
    p = round_to<PD>(p + (s.neg_step * m) / denom);
}

// PD: dtype of p, m, v; GD: dtype of g.  kWriteBack stores the scaled gradient back into
// g whenever a multiply changed it: the clip multiplier differs from 1 (the reference
// multiplies only when its coefficient is below 1) or an unscale factor is pending.
template <int PD, int GD, bool kLerpSmall, bool kUnscale, bool kWriteBack>
__global__ __launch_bounds__(adamw_block<PD>()) void adamw_kernel(AdamTable tab, AdamScalars s,
                                                           const AdamScalars* __restrict__ slot,
                                                           const float* __restrict__ grad_mul,
                                                           int64_t block_base) {
    if (slot != nullptr) s = *slot;
    constexpr int K = adam_vec<PD>();
    constexpr int kBlock = adamw_block<PD>();
    constexpr int kUnroll = adamw_unroll<PD, kWriteBack>();
    constexpr int64_t kTile = adamw_tile<PD, kWriteBack>();
    const int64_t block = block_base + blockIdx.x;
    const int t = owning_tensor(tab.first_block, tab.count, block);
    const int64_t base = (block - tab.first_block[t]) * kTile;
    const int64_t n = tab.n[t];
    const float gmul = grad_mul != nullptr ? *grad_mul : 1.0f;
    const bool write_g = kWriteBack && (kUnscale || gmul != 1.0f);
    void* P = tab.p[t];
    void* G = tab.g[t];
    void* M = tab.m[t];
    void* V = tab.v[t];

    if (tab.vec_ok[t] && base + kTile <= n) {
        float pv[kUnroll][K], gv[kUnroll][K], mv[kUnroll][K], vv[kUnroll][K];
        // One stream at a time, each load waited for before the next stream's is issued,
        // and the gradient written back (when it is) as soon as it is scaled: the fastest
        // of the issue orders tried (both vectors of a stream before a wait, no waits,
        // streams in pairs; the gradient stored first or last among the stores).
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int64_t e = base + (int64_t(u) * kBlock + threadIdx.x) * K;
            load_vec<GD, K>(G, e, gv[u]);
            wait_vmem();
            if (write_g) {
#pragma unroll
                for (int c = 0; c < K; ++c) gv[u][c] = scaled_grad<GD, kUnscale>(gv[u][c], s.unscale, gmul);
                store_vec<GD, K>(G, e, gv[u]);
            }
            load_vec<PD, K>(M, e, mv[u]);
            wait_vmem();
            load_vec<PD, K>(V, e, vv[u]);
            wait_vmem();
            load_vec<PD, K>(P, e, pv[u]);
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
            for (int c = 0; c < K; ++c) {
                if (!write_g) gv[u][c] = scaled_grad<GD, kUnscale>(gv[u][c], s.unscale, gmul);
                adamw_update<PD, kLerpSmall>(pv[u][c], gv[u][c], mv[u][c], vv[u][c], s);
            }
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int64_t e = base + (int64_t(u) * kBlock + threadIdx.x) * K;
            store_vec<PD, K>(M, e, mv[u]);
            store_vec<PD, K>(V, e, vv[u]);
            store_vec<PD, K>(P, e, pv[u]);
        }
    } else {
        const int64_t end = base + kTile < n ? base + kTile : n;
        for (int64_t e = base + threadIdx.x; e < end; e += kBlock) {
            float p = load_one<PD>(P, e), m = load_one<PD>(M, e), v = load_one<PD>(V, e);
            const float g = scaled_grad<GD, kUnscale>(load_one<GD>(G, e), s.unscale, gmul);
            adamw_update<PD, kLerpSmall>(p, g, m, v, s);
            store_one<PD>(P, e, p);
            store_one<PD>(M, e, m);
            store_one<PD>(V, e, v);
            if (write_g) store_one<GD>(G, e, g);
        }
    }
}

// ---- SGD -------------------------------------------------------------------------
// torch's single-tensor SGD (torch/optim/sgd.py, _single_tensor_sgd) per element, with
// the unscale and clip multiplies in front.  Every `x.add(y, alpha=a)` of torch's CPU
// path is one fused multiply-add, fma(y, a, x), whose alpha torch first rounds to the
// tensor's dtype (the host passes the alphas so rounded); mul_ is one rounded multiply
// by the unrounded fp32 scalar.  For a 2-byte PD each op's result is rounded to PD.
enum SgdMode { kSgdPlain = 0, kSgdFirst = 1, kSgdMomentum = 2 };

struct SgdTable {
    void* p[kMaxT];
    void* g[kMaxT];
    void* buf[kMaxT];
    int64_t n[kMaxT];
    int64_t first_block[kMaxT + 1];
    int32_t vec_ok[kMaxT];
    int32_t count;
};

struct SgdScalars {
    float unscale;
    float weight_decay;         // alpha of grad.add(param, alpha=wd)
    float momentum;             // buf.mul_(momentum)
    float momentum_alpha;       // alpha of grad.add(buf, alpha=momentum) (Nesterov)
    float one_minus_dampening;  // alpha of buf.add_(grad, alpha=1 - dampening)
    float neg_lr;               // alpha of param.add_(grad, alpha=-lr)
    int32_t apply_weight_decay;
    int32_t nesterov;
};

template <int PD, int kMode>
__device__ __forceinline__ void sgd_update(float& p, float g, float& buf, const SgdScalars& s) {
    if (s.apply_weight_decay) g = round_to<PD>(__builtin_fmaf(p, s.weight_decay, g));  // grad.add(param, alpha=wd)
    if constexpr (kMode == kSgdFirst) {
        buf = g;  // the buffer starts as a clone of the gradient
    } else if constexpr (kMode == kSgdMomentum) {
        buf = round_to<PD>(buf * s.momentum);
        buf = round_to<PD>(__builtin_fmaf(g, s.one_minus_dampening, buf));  // buf.mul_(m).add_(grad, alpha=1-d)
    }
    if constexpr (kMode != kSgdPlain) g = s.nesterov ? round_to<PD>(__builtin_fmaf(buf, s.momentum_alpha, g)) : buf;
    p = round_to<PD>(__builtin_fmaf(g, s.neg_lr, p));  // param.add_(grad, alpha=-lr)
}

template <int PD, int GD, bool kUnscale, int kMode, bool kWriteBack>
__global__ __launch_bounds__(kAdamBlock) void sgd_kernel(SgdTable tab, SgdScalars s,
                                                         const SgdScalars* __restrict__ slot,
                                                         const float* __restrict__ grad_mul,
                                                         int64_t block_base) {
    if (slot != nullptr) s = *slot;
    constexpr int K = adam_vec<PD>();
    constexpr int kUnroll = adam_unroll<kWriteBack>();
    constexpr int64_t kTile = adam_tile<PD, kWriteBack>();
    const int64_t block = block_base + blockIdx.x;
    const int t = owning_tensor(tab.first_block, tab.count, block);
    const int64_t base = (block - tab.first_block[t]) * kTile;
    const int64_t n = tab.n[t];
    const float gmul = grad_mul != nullptr ? *grad_mul : 1.0f;
    const bool write_g = kWriteBack && (kUnscale || gmul != 1.0f);
    void* P = tab.p[t];
    void* G = tab.g[t];
    void* B = tab.buf[t];
    if (tab.vec_ok[t] && base + kTile <= n) {
        float pv[kUnroll][K], gv[kUnroll][K], bv[kUnroll][K];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int64_t e = base + (int64_t(u) * kAdamBlock + threadIdx.x) * K;
            load_vec<GD, K>(G, e, gv[u]);
            wait_vmem();
            if (write_g) {  // written back as soon as it is scaled, as in adamw_kernel
#pragma unroll
                for (int c = 0; c < K; ++c) gv[u][c] = scaled_grad<GD, kUnscale>(gv[u][c], s.unscale, gmul);
                store_vec<GD, K>(G, e, gv[u]);
            }
            if constexpr (kMode == kSgdMomentum) {
                load_vec<PD, K>(B, e, bv[u]);
                wait_vmem();
            }
            load_vec<PD, K>(P, e, pv[u]);
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
            for (int c = 0; c < K; ++c) {
                if (!write_g) gv[u][c] = scaled_grad<GD, kUnscale>(gv[u][c], s.unscale, gmul);
                float b = kMode == kSgdMomentum ? bv[u][c] : 0.0f;
                sgd_update<PD, kMode>(pv[u][c], gv[u][c], b, s);
                bv[u][c] = b;
            }
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int64_t e = base + (int64_t(u) * kAdamBlock + threadIdx.x) * K;
            if constexpr (kMode != kSgdPlain) store_vec<PD, K>(B, e, bv[u]);
            store_vec<PD, K>(P, e, pv[u]);
        }
    } else {
        const int64_t end = base + kTile < n ? base + kTile : n;
        for (int64_t e = base + threadIdx.x; e < end; e += kAdamBlock) {
            float p = load_one<PD>(P, e), b = kMode == kSgdMomentum ? load_one<PD>(B, e) : 0.0f;
            const float g = scaled_grad<GD, kUnscale>(load_one<GD>(G, e), s.unscale, gmul);
            sgd_update<PD, kMode>(p, g, b, s);
            store_one<PD>(P, e, p);
            if constexpr (kMode != kSgdPlain) store_one<PD>(B, e, b);
            if (write_g) store_one<GD>(G, e, g);
        }
    }
}

// ---- squared norm ------------------------------------------------------------------
// 1024-thread workgroups, each summing one contiguous chunk of 8 tiles; a tile is one
// 16-byte load per lane (4 fp32 or 8 bf16/fp16 gradients).
constexpr int kNormBlock = 1024;
constexpr int kNormTilesPerChunk = 8;
// fp32: tiles whose loads a thread issues together in a whole chunk; 0 is the tile loop,
// which the compiler pipelines by itself.  The pass that also stores the unscaled values
// (kStore) issues four.
template <int GD, bool kStore = false>
constexpr int norm_batch() { return kStore ? 4 : 0; }
template <int GD>
constexpr int norm_vec() { return GD == F32 ? 4 : 8; }
template <int GD>
constexpr int64_t norm_tile() { return int64_t(kNormBlock) * norm_vec<GD>(); }
template <int GD>
constexpr int64_t norm_chunk() { return norm_tile<GD>() * kNormTilesPerChunk; }
// Elements per norm partial: 32768 fp32, 65536 bf16 / fp16, 16384 float64 gradients
// (norm_chunk<F64> is not instantiated: the float64 pass has its own kernel).
inline int64_t norm_chunk_of(int32_t dtype) {
    if (dtype == HBT_DTYPE_F64) return int64_t(kNormBlock) * 2 * kNormTilesPerChunk;
    return dtype == F32 ? norm_chunk<F32>() : norm_chunk<BF16>();
}

struct NormTable {
    const void* g[kMaxT];
    int64_t n[kMaxT];
    double w[kMaxT];
    int64_t first_chunk[kMaxT + 1];
    int32_t vec_ok[kMaxT];
    int32_t count;
};

__device__ __forceinline__ double sq(float x) {
    const double d = static_cast<double>(x);
    return d * d;
}

// ---- two-level order of 2-byte gradients -----------------------------------------------
// A piece is 64 lanes x one 16-byte vector: 512 bf16 / fp16 elements, lane l owning
// elements 8l .. 8l + 7 of it; a chunk is 128 pieces.  Lane sums add the squares in
// element order; a piece's sum is the butterfly (shfl_xor 32, 16, ..., 1) of its lane
// sums; a chunk's partial is the butterfly of s_l + s_(l+64) over lanes l = 0..63, times the
// tensor's weight.  Two passes compute it: the plain norm below (1024 threads per chunk,
// wave w summing pieces 16k + w, k = 0..7), and the in-place unscale fused with it
// (one wave per piece, then one wave per chunk), whose every piece moves 1 KB in and out in
// a workgroup that retires at once.  Both give bitwise the same partials.
constexpr int kPiecesPerChunk = 128;
constexpr int64_t kPieceB16 = 64 * 8;

// acc + x * x in double with one rounding: the square of an fp32 value (24-bit significand,
// exponent range far inside double's) is exact in double, so the fused multiply-add rounds
// exactly where acc + sq(x) rounds, in one instruction.
__device__ __forceinline__ double add_sq(double acc, float x) {
    const double d = static_cast<double>(x);
    return __builtin_fma(d, d, acc);
}


// A lane's eight elements of a piece from element e0 (its first), squared after the
// unscale: vector loads when the whole lane vector lies inside and is aligned.
template <int GD, bool kUnscale>
__device__ __forceinline__ double lane_sq_b16(const void* G, int64_t e0, int64_t n, bool vec, float unscale) {
    double acc = 0.0;
    if (vec) {
        float x[8];
        load_vec<GD, 8>(G, e0, x);
#pragma unroll
        for (int c = 0; c < 8; ++c) acc = add_sq(acc, kUnscale ? round_to<GD>(x[c] * unscale) : x[c]);
    } else {
        for (int c = 0; c < 8 && e0 + c < n; ++c) {
            const float y = load_one<GD>(G, e0 + c);
            acc = add_sq(acc, kUnscale ? round_to<GD>(y * unscale) : y);
        }
    }
    return acc;
}

// The eight piece sums of one wave (pieces 16k + w, a[k] its lane sums) by a reduce-scatter
// butterfly: at stage xor 32 a lane keeps pieces 0-3 or 4-7 and adds its partner's, and so
// on, so each piece's sum is the butterfly's bitwise (the same pairs at every stage, and
// addition commutes) for 10 shuffles instead of 48.  Lane l ends with the sum of piece
// 16 (l >> 3) + w.
__device__ __forceinline__ double piece_sums8(const double (&a)[8], int lane) {
    const bool h5 = lane & 32, h4 = lane & 16, h3 = lane & 8;
    double b[4], c[2];
#pragma unroll
    for (int i = 0; i < 4; ++i) b[i] = (h5 ? a[4 + i] : a[i]) + __shfl_xor(h5 ? a[i] : a[4 + i], 32, 64);
#pragma unroll
    for (int i = 0; i < 2; ++i) c[i] = (h4 ? b[2 + i] : b[i]) + __shfl_xor(h4 ? b[i] : b[2 + i], 16, 64);
    double d = (h3 ? c[1] : c[0]) + __shfl_xor(h3 ? c[0] : c[1], 8, 64);
    d += __shfl_xor(d, 4, 64);
    d += __shfl_xor(d, 2, 64);
    d += __shfl_xor(d, 1, 64);
    return d;
}

// The plain pass for 2-byte gradients: chunk c's partial in the two-level order.
template <int GD, bool kUnscale>
__device__ __forceinline__ void sqnorm_b16_chunk(const NormTable& tab, float unscale, double* __restrict__ partials,
                                                 int64_t chunk) {
    __shared__ double piece_sums[kPiecesPerChunk];
    const int t = owning_tensor(tab.first_chunk, tab.count, chunk);
    const int64_t start = (chunk - tab.first_chunk[t]) * kPieceB16 * kPiecesPerChunk;
    const int64_t n = tab.n[t];
    const void* G = tab.g[t];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    double a[8];
    if (tab.vec_ok[t] && start + kPieceB16 * kPiecesPerChunk <= n) {
        // whole chunk: four pieces' loads in flight before the first is summed
#pragma unroll
        for (int k0 = 0; k0 < 8; k0 += 4) {
            float x[4][8];
#pragma unroll
            for (int k = 0; k < 4; ++k)
                load_vec<GD, 8>(G, start + int64_t((k0 + k) * 16 + w) * kPieceB16 + int64_t(lane) * 8, x[k]);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                a[k0 + k] = 0.0;
#pragma unroll
                for (int c = 0; c < 8; ++c) a[k0 + k] = add_sq(a[k0 + k], kUnscale ? round_to<GD>(x[k][c] * unscale) : x[k][c]);
            }
        }
    } else {
#pragma unroll
        for (int k = 0; k < 8; ++k)
            a[k] = lane_sq_b16<GD, kUnscale>(G, start + int64_t(k * 16 + w) * kPieceB16 + int64_t(lane) * 8, n, false,
                                             unscale);
    }
    const double d = piece_sums8(a, lane);
    if ((lane & 7) == 0) piece_sums[(lane >> 3) * 16 + w] = d;
    __syncthreads();
    if (w == 0) {
        const double s = wave_sum(piece_sums[lane] + piece_sums[lane + 64]);
        if (lane == 0) partials[chunk] = s * tab.w[t];
    }
}

// Workgroup c sums chunk c of the concatenated tensors (8 tiles of one tensor: 32768
// fp32 or 65536 bf16/fp16 elements) into partials[c].  Inside a thread the squares are
// added in element order; threads and waves are combined by the fixed trees of
// block_sum, so the partials, and the sum of them, depend only on the data and the
// numels.  A pending unscale is applied, rounded to the gradient's dtype, before squaring.
// kStore writes each unscaled value back in place as it is squared: the in-place unscale
// and the norm of its result in one pass, with the partials of the norm pass over the
// unscaled tensor (the same loads, the same order).
template <int GD, bool kUnscale, bool kStore = false>
__global__ __launch_bounds__(kNormBlock) void sqnorm_kernel(NormTable tab, float unscale,
                                                            double* __restrict__ partials, int64_t block_base) {
    static_assert(!kStore || kUnscale, "a store without an unscale rewrites the same values");
    static_assert(!kStore || GD == F32, "2-byte gradients unscale in place through unscale_pieces_kernel");
    if constexpr (GD != F32) {
        sqnorm_b16_chunk<GD, kUnscale>(tab, unscale, partials, block_base + blockIdx.x);
    } else {
        constexpr int K = norm_vec<GD>();
        constexpr int64_t kTile = norm_tile<GD>();
        constexpr int64_t kChunk = norm_chunk<GD>();
        const int64_t chunk = block_base + blockIdx.x;
        const int t = owning_tensor(tab.first_chunk, tab.count, chunk);
        const int64_t start = (chunk - tab.first_chunk[t]) * kChunk;
        const int64_t n = tab.n[t];
        const void* G = tab.g[t];
        double acc = 0.0;
        constexpr int kNormBatch = norm_batch<GD, kStore>() > 0 ? norm_batch<GD, kStore>() : 1;
        if (norm_batch<GD, kStore>() > 0 && tab.vec_ok[t] && start + kChunk <= n) {
            // a whole chunk: kNormBatch tiles' loads in flight before the first of them is summed
    #pragma unroll
            for (int k0 = 0; k0 < kNormTilesPerChunk; k0 += kNormBatch) {
                float x[kNormBatch][K];
    #pragma unroll
                for (int k = 0; k < kNormBatch; ++k)
                    load_vec<GD, K>(G, start + int64_t(k0 + k) * kTile + int64_t(threadIdx.x) * K, x[k]);
    #pragma unroll
                for (int k = 0; k < kNormBatch; ++k) {
    #pragma unroll
                    for (int c = 0; c < K; ++c) {
                        float y = x[k][c];
                        if constexpr (kUnscale) y = round_to<GD>(y * unscale);
                        if constexpr (kStore) x[k][c] = y;
                        acc += sq(y);
                    }
                    if constexpr (kStore)
                        store_vec<GD, K>(const_cast<void*>(G), start + int64_t(k0 + k) * kTile + int64_t(threadIdx.x) * K,
                                         x[k]);
                }
            }
            const double block_total = block_sum<kNormBlock>(acc);
            if (threadIdx.x == 0) partials[chunk] = block_total * tab.w[t];
            return;
        }
        for (int k = 0; k < kNormTilesPerChunk; ++k) {
            const int64_t base = start + int64_t(k) * kTile;
            if (base >= n) break;
            if (tab.vec_ok[t] && base + kTile <= n) {
                float x[K];
                load_vec<GD, K>(G, base + int64_t(threadIdx.x) * K, x);
    #pragma unroll
                for (int c = 0; c < K; ++c) {
                    float y = x[c];
                    if constexpr (kUnscale) y = round_to<GD>(y * unscale);
                    if constexpr (kStore) x[c] = y;
                    acc += sq(y);
                }
                if constexpr (kStore) store_vec<GD, K>(const_cast<void*>(G), base + int64_t(threadIdx.x) * K, x);
            } else {
                const int64_t end = base + kTile < n ? base + kTile : n;
                for (int64_t e = base + threadIdx.x; e < end; e += kNormBlock) {
                    float y = load_one<GD>(G, e);
                    if constexpr (kUnscale) y = round_to<GD>(y * unscale);
                    if constexpr (kStore) store_one<GD>(const_cast<void*>(G), e, y);
                    acc += sq(y);
                }
            }
        }
        const double block_total = block_sum<kNormBlock>(acc);
        if (threadIdx.x == 0) partials[chunk] = block_total * tab.w[t];
    }
}

// ---- FSDP gradient local share (optionally fused with the norm partials) ------------
// Writes the rank's gradient shard (sum over ranks, in rank order, of cast(x_q) / divisor
// in the reduce dtype; +0.0 over the padding tail), cast to the master dtype OD, and, in
// the same pass, the squared norm of every 256-element tile of that output.  A second,
// small kernel adds each chunk's tile sums into one partial per norm chunk (32768 fp32 or
// 65536 2-byte elements) of the segments [0, valid) and [valid, shard), the layout the
// norm pass uses, so the optimizer can take them in its place.  Every sum has a fixed
// order: per lane the 4 squares in element order, per tile a butterfly over the 64 lanes,
// per chunk lane l's tiles l, l + 64, ... in order, then a butterfly.
struct ShareRanks {
    const uint8_t* g[HBT_MAX_LOCAL_RANKS];
};
// The no_sync accumulator rows of the reduction that ends the accumulation: row q holds
// rank q's accumulated gradient over this rank's slice, in the reduce dtype.
struct ShareAcc {
    const uint8_t* a[HBT_MAX_LOCAL_RANKS];
};

constexpr int kShareBlock = 64;
constexpr int64_t kShareTile = int64_t(kShareBlock) * 4;  // 256 elements, one wave
template <int OD>
constexpr int tiles_per_norm_chunk() { return static_cast<int>(norm_chunk<OD>() / kShareTile); }  // 128 or 256

// Division by a power of two is exact scaling, so x / d == x * (1 / d) bitwise for
// every x (both are the correctly rounded x * 2^-k); other divisors divide.
template <bool kRecip>
__device__ __forceinline__ float share_div(float x, float divisor, float recip) {
    if constexpr (kRecip) return x * recip;
    return x / divisor;
}

// The reference's AVG reduce-scatter in reduce dtype RD over inputs of dtype ID: the
// gradient is cast to RD unless it already has that dtype (Tensor.to), each division
// and each addition is rounded to RD (torch computes them in fp32 and rounds once).
template <int ID, int RD>
__device__ __forceinline__ float share_cast(float x) {
    if constexpr (ID == RD) return x;
    return round_to<RD>(x);
}

// One wave per 256-element tile, each rank's 512 B of bf16 read by one 8-byte load per
// lane: of the per-wave sizes tried (128 to 512 elements) and the 1024-thread, 8-tile
// workgroups of the norm kernel, this streams fastest, at the rate of a kernel that
// only sums the same eight streams as raw words.  kG > 0 fixes the group size so that
// every rank's load is issued before the first is used; kG == 0 reads group_size at run
// time.  With kG fixed the loads go out in pairs, each pair waited for before the next
// is issued, which beat all eight in flight at once, waiting after each load, and
// waiting after four.  tile_sums may be null (the local share alone).
constexpr int kShareIssue = 2;
// With the accumulator rows (kAcc) each rank is two loads, its gradient and its row;
// waiting after every rank's pair streamed fastest (against every two, four or eight
// ranks, or all gradients before the rows).
constexpr int kShareAccIssue = 1;

// Where tile t's sum is stored among a launch's `tiles` tile sums.  Workgroup b owns
// tile b, and the dispatcher deals consecutive workgroups to the 8 XCDs in turn, each
// with its own L2: stored at index t, every 64-byte line of sums would be written back
// by eight XCDs in eight partial pieces, four times the bytes of the sums.  So the sums
// of the tiles XCD x runs are stored together: within each launch slice of n tiles,
// tile b goes to (b mod 8) * (n / 8) + b / 8 (the last n mod 8 keep their index).
// Giving each XCD a contiguous eighth of the tiles instead fixes the writes as well but
// slowed the launch.  The slot is a bijection, and the reader applies the same one, so
// the partials do not change.
constexpr int kXcds = 8;
__device__ __forceinline__ int64_t tile_sum_slot(int64_t t, int64_t tiles) {
    constexpr int64_t kSlice = kGridMaxItems / kShareBlock;  // launch_sliced's slices
    const int64_t first = (t / kSlice) * kSlice;
    const int64_t n = tiles - first < kSlice ? tiles - first : kSlice;
    const int64_t b = t - first;
    const int64_t per = n / kXcds;
    return first + (b < per * kXcds ? (b % kXcds) * per + b / kXcds : b);
}
// In-place unscale of 2-byte gradients fused with their norm partials, in the two-level
// order of the plain pass: one wave per piece reads its 1 KB, stores the unscaled values,
// then sums their squares and writes the piece sum (slots grouped by XCD, as the tile
// sums are); fold_pieces_kernel then forms each chunk's partial.  Storing before summing
// and retiring after 1 KB keeps the in-place stream at the rate of a plain copy, where
// 1024-thread workgroups holding a chunk each stream about 6% slower.
template <int GD>
__global__ __launch_bounds__(64) void unscale_pieces_kernel(NormTable tab, float unscale,
                                                            double* __restrict__ piece_sums, int64_t pieces,
                                                            int64_t block_base) {
    const int64_t p = block_base + blockIdx.x;
    const int64_t chunk = p / kPiecesPerChunk;
    const int t = owning_tensor(tab.first_chunk, tab.count, chunk);
    const int64_t e0 = (chunk - tab.first_chunk[t]) * kPieceB16 * kPiecesPerChunk +
                       (p % kPiecesPerChunk) * kPieceB16 + int64_t(threadIdx.x) * 8;
    const int64_t n = tab.n[t];
    uint16_t* G = static_cast<uint16_t*>(const_cast<void*>(tab.g[t]));  // written in place
    constexpr bool kHalf = GD == F16;
    double acc = 0.0;
    if (tab.vec_ok[t] && e0 + 8 <= n) {
        // Packed conversions, and the squares taken of the stored values: about 6.5 VALU
        // operations per element, where rounding through round_to and store_vec took 14
        // and left this pass ALU-bound.
        const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(G + e0));
        float y[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            y[2 * i] = b16_to_f32<kHalf>(w[i] & 0xFFFFu) * unscale;
            y[2 * i + 1] = b16_to_f32<kHalf>(w[i] >> 16) * unscale;
        }
        const u32x4 o = pack8_rounded<GD>(y);
        __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(G + e0));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc = add_sq(acc, b16_to_f32<kHalf>(o[i] & 0xFFFFu));
            acc = add_sq(acc, b16_to_f32<kHalf>(o[i] >> 16));
        }
    } else {
        for (int c = 0; c < 8 && e0 + c < n; ++c) {
            const uint32_t r = f32_to_b16<kHalf>(round_to<GD>(b16_to_f32<kHalf>(G[e0 + c]) * unscale));
            G[e0 + c] = static_cast<uint16_t>(r);
            acc = add_sq(acc, b16_to_f32<kHalf>(r));
        }
    }
    acc = wave_sum(acc);
    if (threadIdx.x == 0) piece_sums[tile_sum_slot(p, pieces)] = acc;
}
__global__ __launch_bounds__(64) void fold_pieces_kernel(NormTable tab, const double* __restrict__ piece_sums,
                                                         int64_t pieces, double* __restrict__ partials,
                                                         int64_t block_base) {
    const int64_t chunk = block_base + blockIdx.x;
    const int t = owning_tensor(tab.first_chunk, tab.count, chunk);
    const int64_t p = chunk * kPiecesPerChunk + threadIdx.x;
    const double s = wave_sum(piece_sums[tile_sum_slot(p, pieces)] + piece_sums[tile_sum_slot(p + 64, pieces)]);
    if (threadIdx.x == 0) partials[chunk] = s * tab.w[t];
}

// The value a store to RD and a reload leave: round_to for fp32 and fp16, and for bf16 the
// same rounding with any NaN stored as the canonical 0x7FC0, as f32_to_bf16 stores it.
template <int RD>
__device__ __forceinline__ float stored(float x) {
    if constexpr (RD == BF16) return bf16_to_f32(f32_to_bf16(x));
    return round_to<RD>(x);
}

// Rank q's element in the reduce dtype: the gradient cast to RD and, when kAcc, added to
// the accumulated one as the reference's final no_sync step adds them before reducing,
// formed exactly as accumulate_kernel forms and stores R(acc + R(grad)), so the fused
// reduction equals an accumulate launch followed by a reduction of the rows bit for bit,
// NaNs included.
template <int ID, int RD, bool kAcc>
__device__ __forceinline__ float share_input(float g, float a) {
    const float x = share_cast<ID, RD>(g);
    if constexpr (kAcc) return stored<RD>(a + x);
    return x;
}

// One 256-element tile of the local share, run by the 64 lanes of one wave (`lane` is
// this thread's lane): writes the tile's outputs and returns this lane's part of the tile's
// squared norm.
template <int ID, int kG, bool kRecip, int RD, int OD, bool kAcc>
__device__ __forceinline__ double share_tile(const ShareRanks& ranks, const ShareAcc& accs, int32_t group_size,
                                             int64_t offset, int64_t shard_numel, int64_t valid_numel, float divisor,
                                             float recip, int32_t vec_ok, void* __restrict__ out, int64_t tile,
                                             int lane) {
    constexpr int64_t IB = bytes_of<ID>();
    const int64_t base = tile * kShareTile;
    double acc = 0.0;
    if (vec_ok && base + kShareTile <= valid_numel) {
        const int64_t e = base + int64_t(lane) * 4;
        float sum[4];
        if constexpr (kG > 0) {
            float x[kG][4];
            float a[kAcc ? kG : 1][4];
#pragma unroll
            for (int q = 0; q < kG; ++q) {
                load_vec<ID, 4>(ranks.g[q] + offset * IB, e, x[q]);
                if constexpr (kAcc) load_vec<RD, 4>(accs.a[q], e, a[q]);
                if ((q + 1) % (kAcc ? kShareAccIssue : kShareIssue) == 0 && q + 1 < kG) wait_vmem();
            }
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                sum[c] = round_to<RD>(share_div<kRecip>(share_input<ID, RD, kAcc>(x[0][c], a[0][c]), divisor, recip));
#pragma unroll
                for (int q = 1; q < kG; ++q) {
                    const float xq = share_input<ID, RD, kAcc>(x[q][c], a[kAcc ? q : 0][c]);
                    sum[c] = round_to<RD>(sum[c] + round_to<RD>(share_div<kRecip>(xq, divisor, recip)));
                }
            }
        } else {
            float x[4];
            float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            load_vec<ID, 4>(ranks.g[0] + offset * IB, e, x);
            if constexpr (kAcc) load_vec<RD, 4>(accs.a[0], e, a);
#pragma unroll
            for (int c = 0; c < 4; ++c) sum[c] = round_to<RD>(share_div<kRecip>(share_input<ID, RD, kAcc>(x[c], a[c]), divisor, recip));
            for (int32_t q = 1; q < group_size; ++q) {
                load_vec<ID, 4>(ranks.g[q] + offset * IB, e, x);
                if constexpr (kAcc) load_vec<RD, 4>(accs.a[q], e, a);
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    sum[c] = round_to<RD>(sum[c] + round_to<RD>(share_div<kRecip>(share_input<ID, RD, kAcc>(x[c], a[c]), divisor, recip)));
                }
            }
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) sum[c] = round_to<OD>(sum[c]);
        store_vec<OD, 4>(out, e, sum);
#pragma unroll
        for (int c = 0; c < 4; ++c) acc += sq(sum[c]);
    } else if (vec_ok && base >= valid_numel && base + kShareTile <= shard_numel) {
        const float zero[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        store_vec<OD, 4>(out, base + int64_t(lane) * 4, zero);
    } else {
        const int64_t end = base + kShareTile < shard_numel ? base + kShareTile : shard_numel;
        for (int64_t e = base + lane; e < end; e += kShareBlock) {
            float v = 0.0f;
            if (e < valid_numel) {
                const float a0 = kAcc ? load_one<RD>(accs.a[0], e) : 0.0f;
                v = round_to<RD>(share_div<kRecip>(share_input<ID, RD, kAcc>(load_one<ID>(ranks.g[0], offset + e), a0),
                                                   divisor, recip));
                for (int32_t q = 1; q < group_size; ++q) {
                    const float aq = kAcc ? load_one<RD>(accs.a[q], e) : 0.0f;
                    const float x = share_input<ID, RD, kAcc>(load_one<ID>(ranks.g[q], offset + e), aq);
                    v = round_to<RD>(v + round_to<RD>(share_div<kRecip>(x, divisor, recip)));
                }
                v = round_to<OD>(v);
            }
            store_one<OD>(out, e, v);
            acc += sq(v);
        }
    }
    return acc;
}

template <int ID, int kG, bool kRecip, int RD, int OD, bool kAcc = false>
__global__ __launch_bounds__(kShareBlock) void local_share_tiles_kernel(
    ShareRanks ranks, ShareAcc accs, int32_t group_size, int64_t offset, int64_t shard_numel, int64_t valid_numel,
    float divisor, float recip, int32_t vec_ok, void* __restrict__ out, double* __restrict__ tile_sums,
    int64_t block_base) {
    const int64_t tile = block_base + blockIdx.x;
    double acc = share_tile<ID, kG, kRecip, RD, OD, kAcc>(ranks, accs, group_size, offset, shard_numel, valid_numel,
                                                          divisor, recip, vec_ok, out, tile,
                                                          static_cast<int>(threadIdx.x));
    if (tile_sums == nullptr) return;
    acc = wave_sum(acc);
    if (threadIdx.x == 0) tile_sums[tile_sum_slot(tile, (shard_numel + kShareTile - 1) / kShareTile)] = acc;
}

// A shard of at most kSmallShareTiles tiles and its norm partials in one launch: one
// workgroup with one wave per tile.  Wave w runs tile w as local_share_tiles_kernel runs
// it; wave 0 then forms the partial of the shard's real segment from the tile sums as
// tile_sums_to_partials_kernel does (lane l adds tile l's sum to +0.0, then the butterfly;
// the segment is a single norm chunk) and writes +0.0 for the padding segment, so outputs
// and partials are bitwise the two-launch form's.  A small model's step is bound by launch
// time, and this takes one launch out of it.
constexpr int kSmallShareTiles = 16;

template <int ID, int kG, bool kRecip, int RD, int OD>
__global__ __launch_bounds__(kSmallShareTiles * kShareBlock) void local_share_small_kernel(
    ShareRanks ranks, int32_t group_size, int64_t offset, int64_t shard_numel, int64_t valid_numel, float divisor,
    float recip, int32_t vec_ok, void* __restrict__ out, double* __restrict__ partials) {
    static_assert(kSmallShareTiles <= kShareBlock && kSmallShareTiles <= tiles_per_norm_chunk<OD>(),
                  "a small shard's segments are one norm chunk each");
    __shared__ double sums[kSmallShareTiles];
    const int wave = static_cast<int>(threadIdx.x) / kShareBlock;  // the launch has one wave per tile
    const int lane = static_cast<int>(threadIdx.x) % kShareBlock;
    const ShareAcc none{};
    const double s = wave_sum(share_tile<ID, kG, kRecip, RD, OD, false>(
        ranks, none, group_size, offset, shard_numel, valid_numel, divisor, recip, vec_ok, out, wave, lane));
    if (lane == 0) sums[wave] = s;
    __syncthreads();
    if (wave != 0) return;
    const int64_t valid_tiles = (valid_numel + kShareTile - 1) / kShareTile;
    double acc = 0.0;
    if (lane < valid_tiles) acc += sums[lane];
    acc = wave_sum(acc);
    if (lane == 0) {
        int slot = 0;
        if (valid_numel > 0) partials[slot++] = acc;
        if (shard_numel > valid_numel) partials[slot] = 0.0;
    }
}

// Reduce dtype float64: each rank's element widens exactly to double (IB = 8 reads a
// float64 no_sync accumulator or float64 gradients), the divide and the rank-order sum run
// in double, both correctly rounded as torch's float64 div and add are (a power-of-two
// divisor multiplies by its exact reciprocal, kRecip: the same bits), and the sum narrows
// to the master dtype OD as Tensor.to does: kept for a float64 master, else to fp32
// rounding to nearest even and then, for a 2-byte OD, to OD.  Lane l owns elements
// 4l .. 4l + 3 of its 256-element tile on every path, so a tile's sum of squares has one
// order.  On whole tiles each rank's four elements are one vector load (two for doubles),
// the ranks issued two at a time ahead of their use, and the output is one vector store.
template <int OD>
__device__ __forceinline__ double narrow_from_f64(double s) {
    if constexpr (OD == HBT_DTYPE_F64) return s;
    return static_cast<double>(round_to<OD>(static_cast<float>(s)));
}
template <int OD>
__device__ __forceinline__ void store4_from_f64(void* base, int64_t e, const double (&o)[4]) {
    if constexpr (OD == HBT_DTYPE_F64) {
        store_f64<4>(base, e, o);
    } else {
        const float f[4] = {static_cast<float>(o[0]), static_cast<float>(o[1]), static_cast<float>(o[2]),
                            static_cast<float>(o[3])};  // exact: o already holds OD values
        store_vec<OD, 4>(base, e, f);
    }
}
template <int OD>
__device__ __forceinline__ void store1_from_f64(void* base, int64_t e, double o) {
    if constexpr (OD == HBT_DTYPE_F64) static_cast<double*>(base)[e] = o;
    else store_one<OD>(base, e, static_cast<float>(o));
}
template <bool kRecip>
__device__ __forceinline__ double share_div64(double x, double divisor, double recip) {
    if constexpr (kRecip) return x * recip;
    return x / divisor;
}

template <int IB, bool IH, int OD, bool kRecip, int kG = 0>
__global__ __launch_bounds__(kShareBlock) void local_share_f64_tiles_kernel(
    ShareRanks ranks, int32_t group_size, int64_t offset, int64_t shard_numel, int64_t valid_numel,
    double divisor, double recip, int32_t vec_ok, void* __restrict__ out, double* __restrict__ tile_sums,
    int64_t block_base) {
    const int64_t tile = block_base + blockIdx.x;
    const int64_t first = tile * kShareTile + int64_t(threadIdx.x) * 4;
    double acc = 0.0;
    if (vec_ok && tile * kShareTile + kShareTile <= valid_numel) {
        double s[4];
        if constexpr (kG > 0) {
            // A fixed group of fp32 / 2-byte inputs: every rank's vector is loaded (the
            // loads waited for in pairs, as in local_share_tiles_kernel) before the first
            // is summed, and held in its own width until it is widened.
            static_assert(IB < 8, "float64 inputs take the run-time group path");
            float f[kG][4];
#pragma unroll
            for (int q = 0; q < kG; ++q) {
                load_vec<dtype_of<IB, IH>(), 4>(ranks.g[q] + offset * IB, first, f[q]);
                if ((q + 1) % 2 == 0 && q + 1 < kG) wait_vmem();
            }
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                s[c] = share_div64<kRecip>(static_cast<double>(f[0][c]), divisor, recip);
#pragma unroll
                for (int q = 1; q < kG; ++q) s[c] = s[c] + share_div64<kRecip>(static_cast<double>(f[q][c]), divisor, recip);
            }
        } else {
            double x[4], y[4];
            load4_as_f64<IB, IH>(ranks.g[0] + offset * IB, first, x);
#pragma unroll
            for (int c = 0; c < 4; ++c) s[c] = share_div64<kRecip>(x[c], divisor, recip);
            int32_t q = 1;
            for (; q + 1 < group_size; q += 2) {
                load4_as_f64<IB, IH>(ranks.g[q] + offset * IB, first, x);
                load4_as_f64<IB, IH>(ranks.g[q + 1] + offset * IB, first, y);
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    s[c] = s[c] + share_div64<kRecip>(x[c], divisor, recip);
                    s[c] = s[c] + share_div64<kRecip>(y[c], divisor, recip);
                }
            }
            if (q < group_size) {
                load4_as_f64<IB, IH>(ranks.g[q] + offset * IB, first, x);
#pragma unroll
                for (int c = 0; c < 4; ++c) s[c] = s[c] + share_div64<kRecip>(x[c], divisor, recip);
            }
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            s[c] = narrow_from_f64<OD>(s[c]);
            acc += s[c] * s[c];
        }
        if constexpr (OD == HBT_DTYPE_F64) {
            // A lane's four doubles are 32 contiguous bytes; staged through LDS, each store
            // instruction writes 1 KB contiguous (lane l: elements 2l, 2l + 1 of each half
            // of the tile) instead of every other 16 bytes of 2 KB.
            __shared__ f64x2 stage[2 * kShareBlock];
            stage[2 * threadIdx.x] = f64x2{s[0], s[1]};
            stage[2 * threadIdx.x + 1] = f64x2{s[2], s[3]};
            __syncthreads();
            f64x2* o = reinterpret_cast<f64x2*>(static_cast<double*>(out) + tile * kShareTile);
            __builtin_nontemporal_store(stage[threadIdx.x], o + threadIdx.x);
            __builtin_nontemporal_store(stage[threadIdx.x + kShareBlock], o + kShareBlock + threadIdx.x);
        } else {
            store4_from_f64<OD>(out, first, s);
        }
    } else if (vec_ok && tile * kShareTile >= valid_numel && tile * kShareTile + kShareTile <= shard_numel) {
        const double zero[4] = {0.0, 0.0, 0.0, 0.0};
        store4_from_f64<OD>(out, first, zero);
    } else {
        for (int j = 0; j < 4; ++j) {
            const int64_t e = first + j;
            if (e >= shard_numel) break;
            double v = 0.0;
            if (e < valid_numel) {
                double s = share_div64<kRecip>(widen_f64<IB, IH>(ranks.g[0], offset + e), divisor, recip);
                for (int32_t q = 1; q < group_size; ++q)
                    s = s + share_div64<kRecip>(widen_f64<IB, IH>(ranks.g[q], offset + e), divisor, recip);
                v = narrow_from_f64<OD>(s);
            }
            store1_from_f64<OD>(out, e, v);
            acc += v * v;
        }
    }
    if (tile_sums == nullptr) return;
    acc = wave_sum(acc);
    if (threadIdx.x == 0) tile_sums[tile_sum_slot(tile, (shard_numel + kShareTile - 1) / kShareTile)] = acc;
}

// Chunk c < valid_chunks: the sum of its kTiles tile sums (those below valid_tiles), lane
// l adding tiles l, l + 64, ... in order before the butterfly; padding chunks: 0, the
// square sum of zeros.  `tiles` is the tile count of the launch that wrote the sums
// (their slots, tile_sum_slot); a chunk's sums lie in 8 runs of kTiles / 8 slots.
template <int kTiles>
__global__ __launch_bounds__(kShareBlock) void tile_sums_to_partials_kernel(
    const double* __restrict__ tile_sums, int64_t tiles, int64_t valid_tiles, int64_t valid_chunks,
    double* __restrict__ partials, int64_t block_base) {
    const int64_t chunk = block_base + blockIdx.x;
    double acc = 0.0;
    if (chunk < valid_chunks) {
        const int64_t first = chunk * kTiles + threadIdx.x;
#pragma unroll
        for (int k = 0; k < kTiles / kShareBlock; ++k) {
            const int64_t a = first + int64_t(k) * kShareBlock;
            if (a < valid_tiles) acc += tile_sums[tile_sum_slot(a, tiles)];
        }
    }
    acc = wave_sum(acc);
    if (threadIdx.x == 0) partials[chunk] = acc;
}

constexpr int kFinalBlock = 1024;

__global__ __launch_bounds__(kFinalBlock) void norm_finalize_kernel(
    const double* __restrict__ partials, int64_t count, double max_norm, double* __restrict__ sum_out,
    double* __restrict__ norm_out, float* __restrict__ grad_mul_out, double* __restrict__ grad_mul64_out,
    int32_t* __restrict__ nonfinite_out) {
    // Four independent accumulators per thread keep four loads in flight; they are
    // combined in a fixed order, so the sum stays reproducible.
    double a0 = 0.0, a1 = 0.0, a2 = 0.0, a3 = 0.0;
    int64_t i = threadIdx.x;
    for (; i + 3 * kFinalBlock < count; i += 4 * kFinalBlock) {
        a0 += partials[i];
        a1 += partials[i + kFinalBlock];
        a2 += partials[i + 2 * kFinalBlock];
        a3 += partials[i + 3 * kFinalBlock];
    }
    for (; i < count; i += kFinalBlock) a0 += partials[i];
    const double total = block_sum<kFinalBlock>((a0 + a1) + (a2 + a3));
    if (threadIdx.x != 0) return;
    // clamp_min(0) keeps NaN; sqrt of fp64 is correctly rounded.
    const double clamped = total < 0.0 ? 0.0 : total;
    const double norm = sqrt(clamped);
    if (sum_out != nullptr) sum_out[0] = total;
    if (norm_out != nullptr) norm_out[0] = norm;
    // The reference multiplies by the Python-double coefficient only when it is below 1:
    // fp32, bf16 and fp16 gradients take it as torch passes it to their kernels, rounded
    // to fp32; float64 gradients take the double itself.
    double mul = 1.0;
    if (max_norm > 0.0) {
        const double coef = max_norm / (norm + 1e-6);
        if (coef < 1.0) mul = coef;
    }
    if (grad_mul_out != nullptr) grad_mul_out[0] = static_cast<float>(mul);
    if (grad_mul64_out != nullptr) grad_mul64_out[0] = mul;
    if (nonfinite_out != nullptr) nonfinite_out[0] = isfinite(total) ? 0 : 1;
}

// ---- in-place scaling ---------------------------------------------------------------
// One kilobyte per workgroup, read and written in place: fp32 in half-wave (32-thread)
// workgroups with two 16-byte vectors per lane, bf16/fp16 in full-wave workgroups with
// one vector per lane, packed by pack8_rounded.  A workgroup that retires after 1 KB keeps
// an in-place stream at the rate of a plain copy.
template <int D>
constexpr int scale_block() { return D == F32 ? 32 : 64; }
template <int D>
constexpr int scale_unroll() { return D == F32 ? 2 : 1; }
template <int D>
constexpr int scale_vec() { return D == F32 ? 4 : 8; }
template <int D>
constexpr int64_t scale_tile() { return int64_t(scale_block<D>()) * scale_unroll<D>() * scale_vec<D>(); }

struct ScaleTable {
    void* x[kMaxT];
    int64_t n[kMaxT];
    int64_t first_block[kMaxT + 1];
    int32_t vec_ok[kMaxT];
    int32_t count;
};

// Two separate multiplies, each rounded to D, as two in-place mul_ calls would do.
template <int D>
__device__ __forceinline__ float scale_one(float x, float unscale, float mul) {
    return round_to<D>(round_to<D>(x * unscale) * mul);
}

template <int D>
__global__ __launch_bounds__(64) void scale_kernel(ScaleTable tab, float unscale,
                                                            const float* __restrict__ grad_mul, int64_t block_base) {
    constexpr int K = scale_vec<D>();
    constexpr int kScaleBlock = scale_block<D>();
    constexpr int64_t kTile = scale_tile<D>();
    const float mul = grad_mul != nullptr ? *grad_mul : 1.0f;
    // Both factors 1: nothing to multiply.  The reference's clip multiplies only when its
    // coefficient is below 1, so the gradient is left untouched, bits and all.
    if (unscale == 1.0f && mul == 1.0f) return;
    const int64_t block = block_base + blockIdx.x;
    const int t = owning_tensor(tab.first_block, tab.count, block);
    const int64_t base = (block - tab.first_block[t]) * kTile;
    const int64_t n = tab.n[t];
    void* X = tab.x[t];
    if (tab.vec_ok[t] && base + kTile <= n) {
        if constexpr (D == F32) {
            constexpr int U = scale_unroll<D>();
            float v[U][K];
#pragma unroll
            for (int u = 0; u < U; ++u) load_vec<D, K>(X, base + (int64_t(u) * kScaleBlock + threadIdx.x) * K, v[u]);
#pragma unroll
            for (int u = 0; u < U; ++u) {
#pragma unroll
                for (int c = 0; c < K; ++c) v[u][c] = scale_one<D>(v[u][c], unscale, mul);
                store_vec<D, K>(X, base + (int64_t(u) * kScaleBlock + threadIdx.x) * K, v[u]);
            }
        } else {
            u32x4* P = reinterpret_cast<u32x4*>(static_cast<uint16_t*>(X) + base) + threadIdx.x;
            const u32x4 w = __builtin_nontemporal_load(P);
            float y[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                y[2 * i] = b16_to_f32<D == F16>(w[i] & 0xFFFFu);
                y[2 * i + 1] = b16_to_f32<D == F16>(w[i] >> 16);
            }
            // x * 1 rounds to x (a NaN stays a NaN and is stored as one): the first multiply
            // runs only when it can change a value.
            if (unscale != 1.0f) {
#pragma unroll
                for (int c = 0; c < 8; ++c) y[c] = round_to<D>(y[c] * unscale);
            }
#pragma unroll
            for (int c = 0; c < 8; ++c) y[c] = y[c] * mul;
            __builtin_nontemporal_store(pack8_rounded<D>(y), P);
        }
        return;
    }
    const int64_t end = base + kTile < n ? base + kTile : n;
    for (int64_t i = base + threadIdx.x; i < end; i += kScaleBlock) store_one<D>(X, i, scale_one<D>(load_one<D>(X, i), unscale, mul));
}

// ---- float64 parameters ---------------------------------------------------------------
// With mixed precision off the reference's masters, gradients and optimizer state have the
// parameters' own dtype (parallel/fsdp.py:379-393), float64 included, and torch's optimizers
// step float64 tensors with every Python scalar used as the double it is: nothing is
// rounded to fp32.  These kernels run torch's per-element op sequences in double with
// double scalars, in the shapes of their fp32 counterparts: 32-lane workgroups, one
// stream at a time, 16-byte non-temporal vectors of two doubles, 1 KB per stream per
// workgroup (512 B with the gradient write-back).
constexpr int kF64Vec = 2;
template <bool kWriteBack>
constexpr int64_t adam_f64_tile() { return int64_t(kAdamBlock) * kF64Vec * adam_unroll<kWriteBack>(); }

struct AdamScalarsF64 {
    double unscale;
    double decay;
    double lerp_w;
    double lerp_w_minus_1;
    double beta2;
    double one_minus_beta2;
    double bc2_sqrt;
    double eps;
    double neg_step;
};

// The reference's in-place multiplies on a float64 gradient: the unscale (skipped at 1)
// and the clip, each one rounded double product.
template <bool kUnscale>
__device__ __forceinline__ double scaled_grad64(double g, double unscale, double gmul) {
    if constexpr (kUnscale) g = g * unscale;
    return g * gmul;
}

// torch's _single_tensor_adam on float64 tensors, given the scaled gradient: the fp32
// sequence of adamw_update with every operation in double.
template <bool kLerpSmall>
__device__ __forceinline__ void adamw_update_f64(double& p, double g, double& m, double& v, const AdamScalarsF64& s) {
    p = p * s.decay;
    const double diff = g - m;
    m = kLerpSmall ? __builtin_fma(s.lerp_w, diff, m) : __builtin_fma(s.lerp_w_minus_1, diff, g);
    v = v * s.beta2;
    v = __builtin_fma(s.one_minus_beta2 * g, g, v);
    const double denom = __builtin_sqrt(v) / s.bc2_sqrt + s.eps;
    p = p + (s.neg_step * m) / denom;
}

template <bool kLerpSmall, bool kUnscale, bool kWriteBack>
__global__ __launch_bounds__(kAdamBlock) void adamw_f64_kernel(AdamTable tab, AdamScalarsF64 s,
                                                               const AdamScalarsF64* __restrict__ slot,
                                                               const double* __restrict__ grad_mul,
                                                               int64_t block_base) {
    if (slot != nullptr) s = *slot;
    constexpr int K = kF64Vec;
    constexpr int kUnroll = adam_unroll<kWriteBack>();
    constexpr int64_t kTile = adam_f64_tile<kWriteBack>();
    const int64_t block = block_base + blockIdx.x;
    const int t = owning_tensor(tab.first_block, tab.count, block);
    const int64_t base = (block - tab.first_block[t]) * kTile;
    const int64_t n = tab.n[t];
    const double gmul = grad_mul != nullptr ? *grad_mul : 1.0;
    const bool write_g = kWriteBack && (kUnscale || gmul != 1.0);
    void* P = tab.p[t];
    void* G = tab.g[t];
    void* M = tab.m[t];
    void* V = tab.v[t];
    if (tab.vec_ok[t] && base + kTile <= n) {
        double pv[kUnroll][K], gv[kUnroll][K], mv[kUnroll][K], vv[kUnroll][K];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int64_t e = base + (int64_t(u) * kAdamBlock + threadIdx.x) * K;
            load_f64<K>(G, e, gv[u]);
            wait_vmem();
            if (write_g) {
#pragma unroll
                for (int c = 0; c < K; ++c) gv[u][c] = scaled_grad64<kUnscale>(gv[u][c], s.unscale, gmul);
                store_f64<K>(G, e, gv[u]);
            }
            load_f64<K>(M, e, mv[u]);
            wait_vmem();
            load_f64<K>(V, e, vv[u]);
            wait_vmem();
            load_f64<K>(P, e, pv[u]);
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
            for (int c = 0; c < K; ++c) {
                if (!write_g) gv[u][c] = scaled_grad64<kUnscale>(gv[u][c], s.unscale, gmul);
                adamw_update_f64<kLerpSmall>(pv[u][c], gv[u][c], mv[u][c], vv[u][c], s);
            }
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int64_t e = base + (int64_t(u) * kAdamBlock + threadIdx.x) * K;
            store_f64<K>(M, e, mv[u]);
            store_f64<K>(V, e, vv[u]);
            store_f64<K>(P, e, pv[u]);
        }
    } else {
        const int64_t end = base + kTile < n ? base + kTile : n;
        double* p = static_cast<double*>(P);
        double* g = static_cast<double*>(G);
        double* m = static_cast<double*>(M);
        double* v = static_cast<double*>(V);
        for (int64_t e = base + threadIdx.x; e < end; e += kAdamBlock) {
            double pe = p[e], me = m[e], ve = v[e];
            const double ge = scaled_grad64<kUnscale>(g[e], s.unscale, gmul);
            adamw_update_f64<kLerpSmall>(pe, ge, me, ve, s);
            p[e] = pe;
            m[e] = me;
            v[e] = ve;
            if (write_g) g[e] = ge;
        }
    }
}

struct SgdScalarsF64 {
    double unscale;
    double weight_decay;
    double momentum;
    double one_minus_dampening;
    double neg_lr;
    int32_t apply_weight_decay;
    int32_t nesterov;
};

// torch's _single_tensor_sgd on float64 tensors: each add(.., alpha=) one fused
// multiply-add with the unrounded double alpha, mul_ one rounded product.
template <int kMode>
__device__ __forceinline__ void sgd_update_f64(double& p, double g, double& buf, const SgdScalarsF64& s) {
    if (s.apply_weight_decay) g = __builtin_fma(p, s.weight_decay, g);
    if constexpr (kMode == kSgdFirst) {
        buf = g;
    } else if constexpr (kMode == kSgdMomentum) {
        buf = buf * s.momentum;
        buf = __builtin_fma(g, s.one_minus_dampening, buf);
    }
    if constexpr (kMode != kSgdPlain) g = s.nesterov ? __builtin_fma(buf, s.momentum, g) : buf;
    p = __builtin_fma(g, s.neg_lr, p);
}

template <bool kUnscale, int kMode, bool kWriteBack>
__global__ __launch_bounds__(kAdamBlock) void sgd_f64_kernel(SgdTable tab, SgdScalarsF64 s,
                                                             const SgdScalarsF64* __restrict__ slot,
                                                             const double* __restrict__ grad_mul,
                                                             int64_t block_base) {
    if (slot != nullptr) s = *slot;
    constexpr int K = kF64Vec;
    constexpr int kUnroll = adam_unroll<kWriteBack>();
    constexpr int64_t kTile = adam_f64_tile<kWriteBack>();
    const int64_t block = block_base + blockIdx.x;
    const int t = owning_tensor(tab.first_block, tab.count, block);
    const int64_t base = (block - tab.first_block[t]) * kTile;
    const int64_t n = tab.n[t];
    const double gmul = grad_mul != nullptr ? *grad_mul : 1.0;
    const bool write_g = kWriteBack && (kUnscale || gmul != 1.0);
    void* P = tab.p[t];
    void* G = tab.g[t];
    void* B = tab.buf[t];
    if (tab.vec_ok[t] && base + kTile <= n) {
        double pv[kUnroll][K], gv[kUnroll][K], bv[kUnroll][K];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int64_t e = base + (int64_t(u) * kAdamBlock + threadIdx.x) * K;
            load_f64<K>(G, e, gv[u]);
            wait_vmem();
            if (write_g) {
#pragma unroll
                for (int c = 0; c < K; ++c) gv[u][c] = scaled_grad64<kUnscale>(gv[u][c], s.unscale, gmul);
                store_f64<K>(G, e, gv[u]);
            }
            if constexpr (kMode == kSgdMomentum) {
                load_f64<K>(B, e, bv[u]);
                wait_vmem();
            }
            load_f64<K>(P, e, pv[u]);
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
            for (int c = 0; c < K; ++c) {
                if (!write_g) gv[u][c] = scaled_grad64<kUnscale>(gv[u][c], s.unscale, gmul);
                double b = kMode == kSgdMomentum ? bv[u][c] : 0.0;
                sgd_update_f64<kMode>(pv[u][c], gv[u][c], b, s);
                bv[u][c] = b;
            }
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int64_t e = base + (int64_t(u) * kAdamBlock + threadIdx.x) * K;
            if constexpr (kMode != kSgdPlain) store_f64<K>(B, e, bv[u]);
            store_f64<K>(P, e, pv[u]);
        }
    } else {
        const int64_t end = base + kTile < n ? base + kTile : n;
        double* p = static_cast<double*>(P);
        double* g = static_cast<double*>(G);
        double* bufp = static_cast<double*>(B);
        for (int64_t e = base + threadIdx.x; e < end; e += kAdamBlock) {
            double pe = p[e], b = kMode == kSgdMomentum ? bufp[e] : 0.0;
            const double ge = scaled_grad64<kUnscale>(g[e], s.unscale, gmul);
            sgd_update_f64<kMode>(pe, ge, b, s);
            p[e] = pe;
            if constexpr (kMode != kSgdPlain) bufp[e] = b;
            if (write_g) g[e] = ge;
        }
    }
}

// In-place x = (x * unscale) * (*grad_mul) on float64 tensors, each product rounded in
// double; nothing when both factors are 1.  Half-wave workgroups, two 16-byte vectors
// per lane (128 elements per workgroup, 1 KB).
constexpr int kScaleF64Unroll = 2;
constexpr int64_t kScaleF64Tile = int64_t(32) * kScaleF64Unroll * kF64Vec;
__global__ __launch_bounds__(32) void scale_f64_kernel(ScaleTable tab, double unscale,
                                                       const double* __restrict__ grad_mul, int64_t block_base) {
    const double mul = grad_mul != nullptr ? *grad_mul : 1.0;
    if (unscale == 1.0 && mul == 1.0) return;
    const int64_t block = block_base + blockIdx.x;
    const int t = owning_tensor(tab.first_block, tab.count, block);
    const int64_t base = (block - tab.first_block[t]) * kScaleF64Tile;
    const int64_t n = tab.n[t];
    void* X = tab.x[t];
    if (tab.vec_ok[t] && base + kScaleF64Tile <= n) {
        double v[kScaleF64Unroll][kF64Vec];
#pragma unroll
        for (int u = 0; u < kScaleF64Unroll; ++u) load_f64<kF64Vec>(X, base + (int64_t(u) * 32 + threadIdx.x) * kF64Vec, v[u]);
#pragma unroll
        for (int u = 0; u < kScaleF64Unroll; ++u) {
#pragma unroll
            for (int c = 0; c < kF64Vec; ++c) v[u][c] = (v[u][c] * unscale) * mul;
            store_f64<kF64Vec>(X, base + (int64_t(u) * 32 + threadIdx.x) * kF64Vec, v[u]);
        }
        return;
    }
    const int64_t end = base + kScaleF64Tile < n ? base + kScaleF64Tile : n;
    double* x = static_cast<double*>(X);
    for (int64_t i = base + threadIdx.x; i < end; i += 32) x[i] = (x[i] * unscale) * mul;
}

// Squared norm of float64 gradients: sqnorm_kernel's 1024-thread workgroups, a tile one
// 16-byte vector (two doubles) per lane, eight tiles (16384 elements) per chunk.  Each
// square is one rounded double product, as g.to(float64).pow(2) gives; a thread adds its
// squares in element order and the workgroup combines them with block_sum.  The loads of
// four tiles are issued before the first of them is summed.
constexpr int64_t kNormF64Tile = int64_t(kNormBlock) * kF64Vec;
constexpr int64_t kNormF64Chunk = kNormF64Tile * kNormTilesPerChunk;
__global__ __launch_bounds__(kNormBlock) void sqnorm_f64_kernel(NormTable tab, double* __restrict__ partials,
                                                                int64_t block_base) {
    const int64_t chunk = block_base + blockIdx.x;
    const int t = owning_tensor(tab.first_chunk, tab.count, chunk);
    const int64_t start = (chunk - tab.first_chunk[t]) * kNormF64Chunk;
    const int64_t n = tab.n[t];
    const double* g = static_cast<const double*>(tab.g[t]);
    double acc = 0.0;
    if (tab.vec_ok[t] && start + kNormF64Chunk <= n) {
        constexpr int kBatch = 4;
#pragma unroll
        for (int k0 = 0; k0 < kNormTilesPerChunk; k0 += kBatch) {
            double x[kBatch][kF64Vec];
#pragma unroll
            for (int k = 0; k < kBatch; ++k)
                load_f64<kF64Vec>(g, start + int64_t(k0 + k) * kNormF64Tile + int64_t(threadIdx.x) * kF64Vec, x[k]);
#pragma unroll
            for (int k = 0; k < kBatch; ++k) {
#pragma unroll
                for (int c = 0; c < kF64Vec; ++c) acc += x[k][c] * x[k][c];
            }
        }
    } else {
        for (int k = 0; k < kNormTilesPerChunk; ++k) {
            const int64_t tile = start + int64_t(k) * kNormF64Tile;
            for (int c = 0; c < kF64Vec; ++c) {
                const int64_t e = tile + int64_t(threadIdx.x) * kF64Vec + c;
                if (e < n) acc += g[e] * g[e];
            }
        }
    }
    const double block_total = block_sum<kNormBlock>(acc);
    if (threadIdx.x == 0) partials[chunk] = block_total * tab.w[t];
}

// ---- no_sync gradient accumulation ----------------------------------------------------
// acc = R(acc + R(grad)), R rounding to the accumulator's dtype (the reduce dtype): the
// gradient's cast to that dtype (Tensor.to) and one addition computed in fp32 and
// rounded once (add_).  kAssign writes R(grad) instead: the first micro-batch's clone.
// The scale kernel's shape: half-wave workgroups, two 4-element vectors per lane,
// 256 accumulator elements per workgroup.
constexpr int kAccumBlock = 32;  // half-wave workgroups, two 4-element vectors per lane
constexpr int64_t kAccumTile = int64_t(kAccumBlock) * 2 * 4;

struct AccumTable {
    void* acc[kMaxT];
    const void* grad[kMaxT];
    int64_t n[kMaxT];
    int64_t first_block[kMaxT + 1];
    int32_t vec_ok[kMaxT];
    int32_t count;
};

// GD: the gradient's dtype; AD: the accumulator's.
template <int GD, int AD, bool kAssign>
__global__ __launch_bounds__(kAccumBlock) void accumulate_kernel(AccumTable tab, int64_t block_base) {
    const int64_t block = block_base + blockIdx.x;
    const int t = owning_tensor(tab.first_block, tab.count, block);
    const int64_t base = (block - tab.first_block[t]) * kAccumTile;
    const int64_t n = tab.n[t];
    void* acc = tab.acc[t];
    const void* grad = tab.grad[t];
    if (tab.vec_ok[t] && base + kAccumTile <= n) {
        float a[2][4], g[2][4];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            load_vec<GD, 4>(grad, base + (int64_t(u) * kAccumBlock + threadIdx.x) * 4, g[u]);
#pragma unroll
            for (int c = 0; c < 4; ++c) g[u][c] = share_cast<GD, AD>(g[u][c]);
        }
        if constexpr (!kAssign) {
#pragma unroll
            for (int u = 0; u < 2; ++u) load_vec<AD, 4>(acc, base + (int64_t(u) * kAccumBlock + threadIdx.x) * 4, a[u]);
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            if constexpr (!kAssign) {
#pragma unroll
                for (int c = 0; c < 4; ++c) g[u][c] = round_to<AD>(a[u][c] + g[u][c]);
            }
            store_vec<AD, 4>(acc, base + (int64_t(u) * kAccumBlock + threadIdx.x) * 4, g[u]);
        }
        return;
    }
    const int64_t end = base + kAccumTile < n ? base + kAccumTile : n;
    for (int64_t i = base + threadIdx.x; i < end; i += kAccumBlock) {
        const float g = share_cast<GD, AD>(load_one<GD>(grad, i));
        store_one<AD>(acc, i, kAssign ? g : round_to<AD>(load_one<AD>(acc, i) + g));
    }
}

// Accumulator float64: the gradient widens exactly (Tensor.to) and each add runs in
// double, as add_ on float64 tensors does; kAssign writes the widened gradient.  The
// layout of accumulate_kernel: each lane owns two runs of four elements, each one vector
// load of the gradient and (without kAssign) two 16-byte loads of the accumulator.
template <int SB, bool SH, bool kAssign>
__global__ __launch_bounds__(kAccumBlock) void accumulate_f64_kernel(AccumTable tab, int64_t block_base) {
    const int64_t block = block_base + blockIdx.x;
    const int t = owning_tensor(tab.first_block, tab.count, block);
    const int64_t base = (block - tab.first_block[t]) * kAccumTile;
    const int64_t n = tab.n[t];
    double* __restrict__ acc = static_cast<double*>(tab.acc[t]);
    const unsigned char* __restrict__ grad = static_cast<const unsigned char*>(tab.grad[t]);
    if (tab.vec_ok[t] && base + kAccumTile <= n) {
        double a[2][4], g[2][4];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int64_t e = base + (int64_t(u) * kAccumBlock + threadIdx.x) * 4;
            load4_as_f64<SB, SH>(grad, e, g[u]);
            if constexpr (!kAssign) load_f64<4>(acc, e, a[u]);
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            if constexpr (!kAssign) {
#pragma unroll
                for (int c = 0; c < 4; ++c) g[u][c] = a[u][c] + g[u][c];
            }
            store_f64<4>(acc, base + (int64_t(u) * kAccumBlock + threadIdx.x) * 4, g[u]);
        }
        return;
    }
    const int64_t end = base + kAccumTile < n ? base + kAccumTile : n;
    for (int64_t i = base + threadIdx.x; i < end; i += kAccumBlock) {
        const double g = widen_f64<SB, SH>(grad, i);
        acc[i] = kAssign ? g : acc[i] + g;
    }
}

// ---- host helpers -----------------------------------------------------------------------
inline bool aligned(const void* ptr, uintptr_t bytes) {
    return (reinterpret_cast<uintptr_t>(ptr) % bytes) == 0;
}

// x rounded to a 2-byte dtype and widened back (host side), as torch rounds a Python
// scalar it adds or uses as an alpha on a tensor of that dtype; fp32 is unchanged.
float host_round_to(float x, int32_t dtype) {
    if (dtype == BF16) {
        uint32_t u;
        std::memcpy(&u, &x, sizeof u);
        if ((u & 0x7FFFFFFFu) > 0x7F800000u) return x;
        u += 0x7FFFu + ((u >> 16) & 1u);
        u &= 0xFFFF0000u;
        float y;
        std::memcpy(&y, &u, sizeof y);
        return y;
    }
    if (dtype == F16) return static_cast<float>(static_cast<_Float16>(x));
    return x;
}

// The optimizer dtype pairs (parameter, gradient) with a kernel.
bool optimizer_dtypes_ok(int32_t param_dtype, int32_t grad_dtype) {
    return (param_dtype == F32 && (grad_dtype == F32 || grad_dtype == BF16)) ||
           (param_dtype == BF16 && grad_dtype == BF16) || (param_dtype == F16 && grad_dtype == F16);
}

// The scalars each step kernel receives, built from an entry point's arguments.  The
// step entry points pass them by value; the slot writers store the same records in
// device memory for the slot forms of the steps to read.
AdamScalars adam_scalars(int32_t param_dtype, float unscale, float decay, float lerp_weight, float beta2,
                         float one_minus_beta2, float bias_correction2_sqrt, float eps, float neg_step_size) {
    AdamScalars s{};
    s.unscale = unscale;
    s.decay = decay;
    s.lerp_w = lerp_weight;
    s.lerp_w_minus_1 = lerp_weight - 1.0f;
    s.beta2 = beta2;
    s.one_minus_beta2 = one_minus_beta2;
    s.bc2_sqrt = bias_correction2_sqrt;
    s.eps = host_round_to(eps, param_dtype);
    s.neg_step = neg_step_size;
    return s;
}

// torch rounds each `alpha` (and nothing multiplied by mul_) to the parameter dtype.
SgdScalars sgd_scalars(int32_t param_dtype, float unscale, float weight_decay, float momentum,
                       float one_minus_dampening, float neg_lr, int32_t flags) {
    return SgdScalars{unscale,
                      host_round_to(weight_decay, param_dtype),
                      momentum,
                      host_round_to(momentum, param_dtype),
                      host_round_to(one_minus_dampening, param_dtype),
                      host_round_to(neg_lr, param_dtype),
                      (flags & HBT_SGD_WEIGHT_DECAY) != 0,
                      (flags & HBT_SGD_NESTEROV) != 0};
}

AdamScalarsF64 adam_scalars_f64(double unscale, double decay, double lerp_weight, double beta2,
                                double one_minus_beta2, double bias_correction2_sqrt, double eps,
                                double neg_step_size) {
    return AdamScalarsF64{unscale, decay, lerp_weight, lerp_weight - 1.0, beta2, one_minus_beta2,
                          bias_correction2_sqrt, eps, neg_step_size};
}

SgdScalarsF64 sgd_scalars_f64(double unscale, double weight_decay, double momentum, double one_minus_dampening,
                              double neg_lr, int32_t flags) {
    return SgdScalarsF64{unscale, weight_decay, momentum, one_minus_dampening, neg_lr,
                         (flags & HBT_SGD_WEIGHT_DECAY) != 0, (flags & HBT_SGD_NESTEROV) != 0};
}

// ---- small host-built data into device memory --------------------------------------------
// One launch stores up to kWordsPerWrite 32-bit words that arrive in its arguments, one
// 64-lane block per kWordsPerBlock of them: thread i of the grid stores word i.  The
// argument block lives in the kernarg segment, so each lane reads its word with one
// vector load from there (no scratch copy).  A recorded launch keeps its arguments, so a
// graph replays the write with the words it was given.
constexpr int kWordsPerWrite = 256;
constexpr int kWordsPerBlock = 64;
struct WordBlock {
    uint32_t w[kWordsPerWrite];
};

__global__ __launch_bounds__(kWordsPerBlock) void write_words_kernel(uint32_t* __restrict__ dst, WordBlock words,
                                                                      int32_t count) {
    // The grid has ceil(count / 64) <= 4 blocks and count <= 256, so i < count stays
    // inside the block of words.
    const int i = static_cast<int>(blockIdx.x) * kWordsPerBlock + static_cast<int>(threadIdx.x);
    if (i < count) dst[i] = words.w[i];
}

int32_t write_words(const char* who, void* dst, const uint32_t* words, int64_t count, hipStream_t st) {
    if (count < 0 || (count > 0 && (dst == nullptr || words == nullptr))) {
        set_error("%s: bad destination, words or count (%lld)", who, static_cast<long long>(count));
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if (!aligned(dst, 4)) {
        set_error("%s: the destination must be 4-byte aligned", who);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    for (int64_t first = 0; first < count; first += kWordsPerWrite) {
        const int32_t n = static_cast<int32_t>(count - first < kWordsPerWrite ? count - first : kWordsPerWrite);
        WordBlock block{};
        std::memcpy(block.w, words + first, sizeof(uint32_t) * static_cast<size_t>(n));
        const unsigned blocks = static_cast<unsigned>((n + kWordsPerBlock - 1) / kWordsPerBlock);
        write_words_kernel<<<dim3(blocks), dim3(kWordsPerBlock), 0, st>>>(static_cast<uint32_t*>(dst) + first, block,
                                                                          n);
        const int32_t status = check_launch(who);
        if (status != HBT_OK) return status;
    }
    return HBT_OK;
}

// A scalar record written into a step slot.
template <typename Record>
int32_t write_slot(const char* who, void* slot, const Record& record, hipStream_t st) {
    static_assert(sizeof(Record) % 4 == 0 && sizeof(Record) <= HBT_STEP_SLOT_BYTES, "a record fills part of a slot");
    if (slot == nullptr || !aligned(slot, 16)) {
        set_error("%s: the slot must be non-null, 16-byte aligned device memory", who);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    uint32_t words[sizeof(Record) / 4];
    std::memcpy(words, &record, sizeof(Record));
    return write_words(who, slot, words, static_cast<int64_t>(sizeof(Record) / 4), st);
}

// A scalar record formatted into HBT_STEP_SLOT_BYTES of host memory, zero past its end,
// for a caller that writes several slots at once.
template <typename Record>
int32_t format_slot(const char* who, void* record, const Record& value) {
    static_assert(sizeof(Record) <= HBT_STEP_SLOT_BYTES, "a record fills part of a slot");
    if (record == nullptr) {
        set_error("%s: the record buffer is null", who);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    std::memset(record, 0, HBT_STEP_SLOT_BYTES);
    std::memcpy(record, &value, sizeof(Record));
    return HBT_OK;
}

// The SGD flags a step or a scalar record accepts.
bool sgd_flags_ok(const char* who, int32_t flags) {
    const int32_t known = HBT_SGD_MOMENTUM | HBT_SGD_FIRST_STEP | HBT_SGD_NESTEROV | HBT_SGD_WEIGHT_DECAY |
                          HBT_STEP_WRITE_GRAD;
    if ((flags & ~known) != 0 ||
        ((flags & (HBT_SGD_FIRST_STEP | HBT_SGD_NESTEROV)) != 0 && (flags & HBT_SGD_MOMENTUM) == 0)) {
        set_error("%s: bad flags 0x%x", who, static_cast<unsigned>(flags));
        return false;
    }
    return true;
}

bool slot_ok(const char* who, const void* slot) {
    if (slot == nullptr || !aligned(slot, 16)) {
        set_error("%s: the slot must be non-null, 16-byte aligned device memory", who);
        return false;
    }
    return true;
}

// Validates a gradient table and fills the norm kernel's table; `chunks` is the number
// of partials the launch writes.
int32_t build_norm_table(const char* who, const void* const* grads, const int64_t* numels,
                         const double* weights, int32_t count, int32_t grad_dtype, NormTable& tab,
                         int64_t& chunks) {
    if (count < 0 || count > kMaxT) {
        set_error("%s: count must lie in [0, %d], got %d", who, kMaxT, count);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if (grad_dtype != F32 && grad_dtype != BF16 && grad_dtype != F16 && grad_dtype != HBT_DTYPE_F64) {
        set_error("%s: gradient dtype %d is not F32, BF16, F16 or F64", who, grad_dtype);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if (count > 0 && (grads == nullptr || numels == nullptr || weights == nullptr)) {
        set_error("%s: null pointer argument", who);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    tab = NormTable{};
    tab.count = count;
    const int64_t kChunk = norm_chunk_of(grad_dtype);
    chunks = 0;
    for (int i = 0; i < count; ++i) {
        if (numels[i] < 0 || (numels[i] > 0 && grads[i] == nullptr)) {
            set_error("%s: tensor %d has a bad pointer or numel", who, i);
            return HBT_ERR_INVALID_ARGUMENT;
        }
        tab.g[i] = grads[i];
        tab.n[i] = numels[i];
        tab.w[i] = weights[i];
        tab.vec_ok[i] = aligned(grads[i], 16);
        tab.first_chunk[i] = chunks;
        chunks += (numels[i] + kChunk - 1) / kChunk;
    }
    tab.first_chunk[count] = chunks;
    for (int i = count + 1; i <= kMaxT; ++i) tab.first_chunk[i] = chunks;
    return HBT_OK;
}

// sqnorm_kernel launches writing partials[0, chunks).
// With `store`, the unscaled values are also written back (nothing to write for unscale 1);
// 2-byte gradients then run unscale_pieces_kernel + fold_pieces_kernel, with
// kPiecesPerChunk * chunks doubles of piece_scratch.
int32_t launch_sqnorm(const char* who, const NormTable& tab, int64_t chunks, int32_t grad_dtype, float unscale,
                      double* partials, hipStream_t st, bool store = false, double* piece_scratch = nullptr) {
    const bool scaled = unscale != 1.0f;
    if (scaled && store && grad_dtype != F32 && grad_dtype != HBT_DTYPE_F64) {
        const int64_t pieces = chunks * kPiecesPerChunk;
        const int32_t status = launch_sliced(who, pieces, 64, [&](int64_t first, dim3 grid) {
            if (grad_dtype == BF16)
                unscale_pieces_kernel<BF16><<<grid, 64, 0, st>>>(tab, unscale, piece_scratch, pieces, first);
            else
                unscale_pieces_kernel<F16><<<grid, 64, 0, st>>>(tab, unscale, piece_scratch, pieces, first);
        });
        if (status != HBT_OK) return status;
        return launch_sliced(who, chunks, 64, [&](int64_t first, dim3 grid) {
            fold_pieces_kernel<<<grid, 64, 0, st>>>(tab, piece_scratch, pieces, partials, first);
        });
    }
    if (grad_dtype == HBT_DTYPE_F64) {
        // The callers refuse a float64 unscale or store: the multiply belongs in double.
        return launch_sliced(who, chunks, kNormBlock, [&](int64_t first, dim3 grid) {
            sqnorm_f64_kernel<<<grid, kNormBlock, 0, st>>>(tab, partials, first);
        });
    }
    return launch_sliced(who, chunks, kNormBlock, [&](int64_t first, dim3 grid) {
        if (grad_dtype == F32) {
            if (scaled && store) sqnorm_kernel<F32, true, true><<<grid, kNormBlock, 0, st>>>(tab, unscale, partials, first);
            else if (scaled) sqnorm_kernel<F32, true><<<grid, kNormBlock, 0, st>>>(tab, unscale, partials, first);
            else sqnorm_kernel<F32, false><<<grid, kNormBlock, 0, st>>>(tab, unscale, partials, first);
        } else if (grad_dtype == BF16) {
            if (scaled) sqnorm_kernel<BF16, true><<<grid, kNormBlock, 0, st>>>(tab, unscale, partials, first);
            else sqnorm_kernel<BF16, false><<<grid, kNormBlock, 0, st>>>(tab, unscale, partials, first);
        } else {
            if (scaled) sqnorm_kernel<F16, true><<<grid, kNormBlock, 0, st>>>(tab, unscale, partials, first);
            else sqnorm_kernel<F16, false><<<grid, kNormBlock, 0, st>>>(tab, unscale, partials, first);
        }
    });
}

// ---- device address of the no-allocation norm's static scratch ------------------------
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
double* g_scratch_ptr[kMaxScratchDevices] = {};

// The device address of this device's copy of `scratch` (looked up on the first call per
// device, with that device current).
int32_t noalloc_scratch(const char* who, double** out) {
    int device = -1;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return check_hip(e, who);
    if (device < 0 || device >= kMaxScratchDevices) {
        set_error("%s: device %d is beyond the %d devices the scratch table covers", who, device,
                  kMaxScratchDevices);
        return HBT_ERR_UNSUPPORTED;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[device] == nullptr) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return check_hip(e, who);
        if (ptr == nullptr) {
            set_error("%s: hipGetSymbolAddress returned a null scratch address", who);
            return HBT_ERR_HIP;
        }
        g_scratch_ptr[device] = static_cast<double*>(ptr);
    }
    *out = g_scratch_ptr[device];
    return HBT_OK;
}

// Shared by hbt_grad_local_share, hbt_grad_local_share_sqnorm (tile_scratch and
// partials null for the former) and hbt_grad_local_share_accumulated (accumulators
// non-null: row q, in the reduce dtype, is added to rank q's gradient first).
int32_t local_share(const char* who, const void* const* rank_grads, int32_t group_size, int32_t rank,
                    int64_t shard_numel, int64_t valid_numel, int32_t in_dtype, int32_t reduce_dtype,
                    float divisor, int32_t out_dtype, void* out, double* partials, double* tile_scratch,
                    hipStream_t st, const void* const* accumulators = nullptr) {
    if (rank_grads == nullptr || out == nullptr || group_size < 1 || group_size > HBT_MAX_LOCAL_RANKS ||
        rank < 0 || rank >= group_size || shard_numel < 0 || valid_numel < 0 || valid_numel > shard_numel) {
        set_error("%s: bad arguments (group_size=%d rank=%d shard=%lld valid=%lld)", who, group_size, rank,
                  static_cast<long long>(shard_numel), static_cast<long long>(valid_numel));
        return HBT_ERR_INVALID_ARGUMENT;
    }
    const bool f64 = reduce_dtype == HBT_DTYPE_F64;
    if (in_dtype != F32 && in_dtype != BF16 && in_dtype != F16 && !(f64 && in_dtype == HBT_DTYPE_F64)) {
        set_error("%s: input dtype %d is not F32, BF16 or F16 (or F64 with reduce dtype F64)", who, in_dtype);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if (reduce_dtype != F32 && reduce_dtype != BF16 && reduce_dtype != F16 && !f64) {
        set_error("%s: reduce dtype %d is not F32, BF16, F16 or F64", who, reduce_dtype);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if (out_dtype != F32 && out_dtype != BF16 && out_dtype != F16 && !(f64 && out_dtype == HBT_DTYPE_F64)) {
        set_error("%s: output (master) dtype %d is not F32, BF16 or F16 (or F64 with reduce dtype F64)", who,
                  out_dtype);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    const bool with_acc = accumulators != nullptr;
    if (with_acc && f64) {
        set_error("%s: an accumulated reduction in reduce dtype F64 is not fused; add the last micro-batch "
                  "with hbt_grad_accumulate and reduce the accumulator", who);
        return HBT_ERR_UNSUPPORTED;
    }
    ShareRanks ranks{};
    ShareAcc accs{};
    const int elem = dtype_size(in_dtype);
    const int64_t offset = int64_t(rank) * shard_numel;
    int32_t vec_ok = aligned(out, 4 * static_cast<uintptr_t>(dtype_size(out_dtype)));
    for (int q = 0; q < group_size; ++q) {
        if (rank_grads[q] == nullptr && valid_numel > 0) {
            set_error("%s: rank %d gradient pointer is null", who, q);
            return HBT_ERR_INVALID_ARGUMENT;
        }
        ranks.g[q] = static_cast<const uint8_t*>(rank_grads[q]);
        const uintptr_t a = reinterpret_cast<uintptr_t>(ranks.g[q]) + static_cast<uintptr_t>(offset * elem);
        if ((a & static_cast<uintptr_t>(4 * elem - 1)) != 0) vec_ok = 0;
        if (with_acc) {
            if (accumulators[q] == nullptr && valid_numel > 0) {
                set_error("%s: rank %d accumulator pointer is null", who, q);
                return HBT_ERR_INVALID_ARGUMENT;
            }
            accs.a[q] = static_cast<const uint8_t*>(accumulators[q]);
            if (!aligned(accs.a[q], 4 * static_cast<uintptr_t>(dtype_size(reduce_dtype)))) vec_ok = 0;
        }
    }
    const int64_t tiles = (shard_numel + kShareTile - 1) / kShareTile;
    if (tiles == 0) return HBT_OK;
    // An exact power of two (or 1) divides as a multiply by its exact reciprocal.
    const float recip = exact_reciprocal(divisor);
    const bool recip_exact = recip != 0.0f;
    // A small shard's share and partials take one launch (local_share_small_kernel).
    const bool small = partials != nullptr && !with_acc && !f64 && tiles <= kSmallShareTiles;
    const unsigned small_threads = static_cast<unsigned>(tiles) * kShareBlock;
    int32_t status = launch_sliced(who, tiles, kShareBlock, [&](int64_t first, dim3 grid) {
#define HBT_TILES(ID, G, R, RD, OD)                                                                             \
    do {                                                                                                       \
        if (small)                                                                                             \
            local_share_small_kernel<ID, G, R, RD, OD><<<dim3(1), dim3(small_threads), 0, st>>>(                 \
                ranks, group_size, offset, shard_numel, valid_numel, divisor, recip, vec_ok, out, partials);    \
        else if (with_acc)                                                                                     \
            local_share_tiles_kernel<ID, G, R, RD, OD, true><<<grid, kShareBlock, 0, st>>>(                      \
                ranks, accs, group_size, offset, shard_numel, valid_numel, divisor, recip, vec_ok, out,          \
                tile_scratch, first);                                                                          \
        else                                                                                                   \
            local_share_tiles_kernel<ID, G, R, RD, OD, false><<<grid, kShareBlock, 0, st>>>(                     \
                ranks, accs, group_size, offset, shard_numel, valid_numel, divisor, recip, vec_ok, out,          \
                tile_scratch, first);                                                                          \
    } while (0)
// The fp32 reduction into an fp32 master has group-size specialisations (the measured
// configuration); other reduce and master dtypes run the run-time group size kernel.
#define HBT_TILES_G(ID, R)                                       \
    do {                                                         \
        switch (group_size) {                                    \
            case 1: HBT_TILES(ID, 1, R, F32, F32); break;        \
            case 2: HBT_TILES(ID, 2, R, F32, F32); break;        \
            case 4: HBT_TILES(ID, 4, R, F32, F32); break;        \
            case 8: HBT_TILES(ID, 8, R, F32, F32); break;        \
            default: HBT_TILES(ID, 0, R, F32, F32); break;       \
        }                                                        \
    } while (0)
#define HBT_TILES_OD(ID, R, RD)                                    \
    do {                                                           \
        if (out_dtype == F32) HBT_TILES(ID, 0, R, RD, F32);        \
        else if (out_dtype == BF16) HBT_TILES(ID, 0, R, RD, BF16); \
        else HBT_TILES(ID, 0, R, RD, F16);                         \
    } while (0)
#define HBT_TILES_RD(ID, R)                                              \
    do {                                                                 \
        if (reduce_dtype == F32 && out_dtype == F32) HBT_TILES_G(ID, R); \
        else if (reduce_dtype == F32) HBT_TILES_OD(ID, R, F32);          \
        else if (reduce_dtype == BF16) HBT_TILES_OD(ID, R, BF16);        \
        else HBT_TILES_OD(ID, R, F16);                                   \
    } while (0)
#define HBT_TILES64G(IB, IH, OD, R, G)                                                                    \
    local_share_f64_tiles_kernel<IB, IH, OD, R, G><<<grid, kShareBlock, 0, st>>>(                          \
        ranks, group_size, offset, shard_numel, valid_numel, static_cast<double>(divisor),                 \
        static_cast<double>(recip), vec_ok, out, tile_scratch, first)
// Groups of 8 narrower inputs have their own instantiation (the measured configuration).
#define HBT_TILES64R(IB, IH, OD, R)                                        \
    do {                                                                   \
        if (IB < 8 && group_size == 8) HBT_TILES64G(IB, IH, OD, R, (IB < 8 ? 8 : 0)); \
        else HBT_TILES64G(IB, IH, OD, R, 0);                               \
    } while (0)
#define HBT_TILES64(IB, IH, OD)                                \
    do {                                                       \
        if (recip_exact) HBT_TILES64R(IB, IH, OD, true);       \
        else HBT_TILES64R(IB, IH, OD, false);                  \
    } while (0)
#define HBT_TILES64_OD(IB, IH)                                                 \
    do {                                                                       \
        if (out_dtype == HBT_DTYPE_F64) HBT_TILES64(IB, IH, HBT_DTYPE_F64);    \
        else if (out_dtype == F32) HBT_TILES64(IB, IH, F32);                   \
        else if (out_dtype == BF16) HBT_TILES64(IB, IH, BF16);                 \
        else HBT_TILES64(IB, IH, F16);                                         \
    } while (0)
        if (f64) {
            if (in_dtype == HBT_DTYPE_F64) HBT_TILES64_OD(8, false);
            else if (in_dtype == F32) HBT_TILES64_OD(4, false);
            else if (in_dtype == BF16) HBT_TILES64_OD(2, false);
            else HBT_TILES64_OD(2, true);
        } else if (in_dtype == F32) {
            if (recip_exact) HBT_TILES_RD(F32, true); else HBT_TILES_RD(F32, false);
        } else if (in_dtype == BF16) {
            if (recip_exact) HBT_TILES_RD(BF16, true); else HBT_TILES_RD(BF16, false);
        } else {
            if (recip_exact) HBT_TILES_RD(F16, true); else HBT_TILES_RD(F16, false);
        }
#undef HBT_TILES64_OD
#undef HBT_TILES64
#undef HBT_TILES64R
#undef HBT_TILES64G
#undef HBT_TILES_RD
#undef HBT_TILES_OD
#undef HBT_TILES_G
#undef HBT_TILES
    });
    if (status != HBT_OK || partials == nullptr || small) return status;
    const int64_t chunk = norm_chunk_of(out_dtype);
    const int64_t valid_chunks = (valid_numel + chunk - 1) / chunk;
    const int64_t pad_chunks = (shard_numel - valid_numel + chunk - 1) / chunk;
    const int64_t valid_tiles = (valid_numel + kShareTile - 1) / kShareTile;
    return launch_sliced(who, valid_chunks + pad_chunks, kShareBlock, [&](int64_t first, dim3 grid) {
        if (out_dtype == HBT_DTYPE_F64) {
            static_assert(kNormF64Chunk % kShareTile == 0, "a float64 norm chunk is whole tiles");
            tile_sums_to_partials_kernel<static_cast<int>(kNormF64Chunk / kShareTile)><<<grid, kShareBlock, 0, st>>>(
                tile_scratch, tiles, valid_tiles, valid_chunks, partials, first);
        } else if (out_dtype == F32) {
            tile_sums_to_partials_kernel<tiles_per_norm_chunk<F32>()><<<grid, kShareBlock, 0, st>>>(
                tile_scratch, tiles, valid_tiles, valid_chunks, partials, first);
        } else {
            tile_sums_to_partials_kernel<tiles_per_norm_chunk<BF16>()><<<grid, kShareBlock, 0, st>>>(
                tile_scratch, tiles, valid_tiles, valid_chunks, partials, first);
        }
    });
}

}  // namespace
}  // namespace hbt

using namespace hbt;

extern "C" {

static int32_t adamw_step_impl(const char* who, void* const* params, void* const* grads, void* const* exp_avgs,
                       void* const* exp_avg_sqs, const int64_t* numels, int32_t count,
                       int32_t param_dtype, int32_t grad_dtype, float unscale, const float* grad_mul,
                       float decay, float lerp_weight, float beta2, float one_minus_beta2,
                       float bias_correction2_sqrt, float eps, float neg_step_size, const AdamScalars* slot, int32_t flags,
                       void* stream) {
    clear_error();
    if (count < 0 || count > kMaxT) {
        set_error("%s: count must lie in [0, %d], got %d", who, kMaxT, count);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if (!optimizer_dtypes_ok(param_dtype, grad_dtype)) {
        set_error("%s: (parameter, gradient) dtypes (%d, %d) are not (F32, F32), (F32, BF16), "
                  "(BF16, BF16) or (F16, F16)", who, param_dtype, grad_dtype);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if ((flags & ~HBT_STEP_WRITE_GRAD) != 0) {
        set_error("%s: unknown flags 0x%x", who, static_cast<unsigned>(flags));
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if (count > 0 && (params == nullptr || grads == nullptr || exp_avgs == nullptr ||
                      exp_avg_sqs == nullptr || numels == nullptr)) {
        set_error("%s: null table pointer", who);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    AdamTable tab{};
    tab.count = count;
    const bool write_back = (flags & HBT_STEP_WRITE_GRAD) != 0;
    const int64_t tile = adamw_tile_of(param_dtype, write_back);
    const int vec = param_dtype == F32 ? adam_vec<F32>() : adam_vec<BF16>();
    const uintptr_t state_align = static_cast<uintptr_t>(vec * dtype_size(param_dtype));
    const uintptr_t grad_align = static_cast<uintptr_t>(vec * dtype_size(grad_dtype));
    int64_t blocks = 0;
    for (int i = 0; i < count; ++i) {
        if (numels[i] < 0) {
            set_error("%s: tensor %d has negative numel %lld", who, i,
                      static_cast<long long>(numels[i]));
            return HBT_ERR_INVALID_ARGUMENT;
        }
        if (numels[i] > 0 && (params[i] == nullptr || grads[i] == nullptr || exp_avgs[i] == nullptr ||
                              exp_avg_sqs[i] == nullptr)) {
            set_error("%s: tensor %d has a null data pointer", who, i);
            return HBT_ERR_INVALID_ARGUMENT;
        }
        tab.p[i] = params[i];
        tab.g[i] = grads[i];
        tab.m[i] = exp_avgs[i];
        tab.v[i] = exp_avg_sqs[i];
        tab.n[i] = numels[i];
        tab.vec_ok[i] = aligned(params[i], state_align) && aligned(grads[i], grad_align) &&
                        aligned(exp_avgs[i], state_align) && aligned(exp_avg_sqs[i], state_align);
        tab.first_block[i] = blocks;
        blocks += (numels[i] + tile - 1) / tile;
    }
    tab.first_block[count] = blocks;
    for (int i = count + 1; i <= kMaxT; ++i) tab.first_block[i] = blocks;
    const AdamScalars s = adam_scalars(param_dtype, unscale, decay, lerp_weight, beta2, one_minus_beta2,
                                       bias_correction2_sqrt, eps, neg_step_size);
    const bool lerp_small = std::fabs(lerp_weight) < 0.5f;
    const bool scaled = unscale != 1.0f;
    hipStream_t st = as_stream(stream);
    return launch_sliced(who, blocks, adamw_block_of(param_dtype), [&](int64_t first, dim3 grid) {
#define HBT_ADAMW(PD, GD, SMALL, SCALED, WB) \
    adamw_kernel<PD, GD, SMALL, SCALED, WB><<<grid, adamw_block<PD>(), 0, st>>>(tab, s, slot, grad_mul, first)
#define HBT_ADAMW_WB(PD, GD, SMALL, SCALED)                     \
    do {                                                        \
        if (write_back) HBT_ADAMW(PD, GD, SMALL, SCALED, true); \
        else HBT_ADAMW(PD, GD, SMALL, SCALED, false);           \
    } while (0)
#define HBT_ADAMW_SCALED(PD, GD, SMALL)                \
    do {                                               \
        if (scaled) HBT_ADAMW_WB(PD, GD, SMALL, true); \
        else HBT_ADAMW_WB(PD, GD, SMALL, false);       \
    } while (0)
#define HBT_ADAMW_LERP(PD, GD)                          \
    do {                                                \
        if (lerp_small) HBT_ADAMW_SCALED(PD, GD, true); \
        else HBT_ADAMW_SCALED(PD, GD, false);           \
    } while (0)
        if (param_dtype == F32 && grad_dtype == F32) HBT_ADAMW_LERP(F32, F32);
        else if (param_dtype == F32) HBT_ADAMW_LERP(F32, BF16);
        else if (param_dtype == BF16) HBT_ADAMW_LERP(BF16, BF16);
        else HBT_ADAMW_LERP(F16, F16);
#undef HBT_ADAMW_LERP
#undef HBT_ADAMW_SCALED
#undef HBT_ADAMW_WB
#undef HBT_ADAMW
    });
}

int64_t hbt_norm_partials_count(const int64_t* numels, int32_t count, int32_t grad_dtype) {
    if (count < 0 || count > kMaxT || (count > 0 && numels == nullptr)) return -1;
    if (grad_dtype != F32 && grad_dtype != BF16 && grad_dtype != F16 && grad_dtype != HBT_DTYPE_F64) return -1;
    const int64_t chunk = norm_chunk_of(grad_dtype);
    int64_t chunks = 0;
    for (int i = 0; i < count; ++i) {
        if (numels[i] < 0) return -1;
        chunks += (numels[i] + chunk - 1) / chunk;
    }
    return chunks;
}

int32_t hbt_grad_sqnorm_partials(const void* const* grads, const int64_t* numels,
                                 const double* weights, int32_t count, int32_t grad_dtype,
                                 float unscale, double* partials, void* stream) {
    clear_error();
    if (count > 0 && partials == nullptr) {
        set_error("hbt_grad_sqnorm_partials: null partials pointer");
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if (grad_dtype == HBT_DTYPE_F64 && unscale != 1.0f) {
        set_error("hbt_grad_sqnorm_partials: float64 gradients are unscaled in double first "
                  "(hbt_scale_inplace_f64); the norm takes unscale 1");
        return HBT_ERR_UNSUPPORTED;
    }
    NormTable tab{};
    int64_t chunks = 0;
    const int32_t status = build_norm_table("hbt_grad_sqnorm_partials", grads, numels, weights, count,
                                            grad_dtype, tab, chunks);
    if (status != HBT_OK) return status;
    return launch_sqnorm("hbt_grad_sqnorm_partials", tab, chunks, grad_dtype, unscale, partials,
                         as_stream(stream));
}

int32_t hbt_scale_inplace_sqnorm(void* const* tensors, const int64_t* numels, int32_t count, int32_t dtype,
                                 float unscale, double* partials, double* piece_scratch, void* stream) {
    clear_error();
    if (count > 0 && partials == nullptr) {
        set_error("hbt_scale_inplace_sqnorm: null partials pointer");
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if (count > 0 && piece_scratch == nullptr && (dtype == BF16 || dtype == F16) && unscale != 1.0f) {
        set_error("hbt_scale_inplace_sqnorm: 2-byte gradients need the piece scratch");
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if (count > 0 && tensors == nullptr) {
        set_error("hbt_scale_inplace_sqnorm: null tensor table");
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if (dtype == HBT_DTYPE_F64) {
        set_error("hbt_scale_inplace_sqnorm: float64 tensors scale in double (hbt_scale_inplace_f64), then "
                  "hbt_grad_sqnorm_partials");
        return HBT_ERR_UNSUPPORTED;
    }
    double ones[kMaxT];
    for (int i = 0; i < kMaxT; ++i) ones[i] = 1.0;
    const void* grads[kMaxT] = {};
    for (int i = 0; i < count && i < kMaxT; ++i) grads[i] = tensors[i];
    NormTable tab{};
    int64_t chunks = 0;
    const int32_t status = build_norm_table("hbt_scale_inplace_sqnorm", count > 0 ? grads : nullptr, numels, ones,
                                            count, dtype, tab, chunks);
    if (status != HBT_OK) return status;
    return launch_sqnorm("hbt_scale_inplace_sqnorm", tab, chunks, dtype, unscale, partials, as_stream(stream),
                         /*store=*/true, piece_scratch);
}

int32_t hbt_grad_norm_finalize(const double* partials, int64_t count, double max_norm,
                               double* sum_out, double* norm_out, float* grad_mul_out,
                               double* grad_mul64_out, int32_t* nonfinite_out, void* stream) {
    clear_error();
    if (count < 0 || (count > 0 && partials == nullptr)) {
        set_error("hbt_grad_norm_finalize: bad partials/count");
        return HBT_ERR_INVALID_ARGUMENT;
    }
    norm_finalize_kernel<<<1, kFinalBlock, 0, as_stream(stream)>>>(partials, count, max_norm, sum_out, norm_out,
                                                                   grad_mul_out, grad_mul64_out, nonfinite_out);
    return check_launch("hbt_grad_norm_finalize");
}

int32_t hbt_grad_norm_noalloc(const void* const* grads, const int64_t* numels, const double* weights,
                              int32_t count, int32_t grad_dtype, float unscale, double max_norm,
                              double* sum_out, double* norm_out, float* grad_mul_out,
                              int32_t* nonfinite_out, void* stream) {
    clear_error();
    if (grad_dtype == HBT_DTYPE_F64) {
        set_error("hbt_grad_norm_noalloc: float64 gradients are not covered (their clip multiplier is a "
                  "double; use hbt_grad_sqnorm_partials + hbt_grad_norm_finalize)");
        return HBT_ERR_UNSUPPORTED;
    }
    NormTable tab{};
    int64_t chunks = 0;
    int32_t status = build_norm_table("hbt_grad_norm_noalloc", grads, numels, weights, count, grad_dtype,
                                      tab, chunks);
    if (status != HBT_OK) return status;
    if (chunks > HBT_NOALLOC_MAX_PARTIALS) {
        set_error("hbt_grad_norm_noalloc: the gradients need %lld norm partials, more than the %d the "
                  "static scratch holds (at most %lld fp32 or %lld bf16/fp16 elements per call)",
                  static_cast<long long>(chunks), HBT_NOALLOC_MAX_PARTIALS,
                  static_cast<long long>(HBT_NOALLOC_MAX_PARTIALS * norm_chunk<F32>()),
                  static_cast<long long>(HBT_NOALLOC_MAX_PARTIALS * norm_chunk<BF16>()));
        return HBT_ERR_UNSUPPORTED;
    }
    double* partials = nullptr;
    status = noalloc_scratch("hbt_grad_norm_noalloc", &partials);
    if (status != HBT_OK) return status;
    hipStream_t st = as_stream(stream);
    // Every slot below `chunks` is written by the norm kernel before the finalize
    // kernel reads it, so the array needs no clearing between calls.
    status = launch_sqnorm("hbt_grad_norm_noalloc", tab, chunks, grad_dtype, unscale, partials, st);
    if (status != HBT_OK) return status;
    norm_finalize_kernel<<<1, kFinalBlock, 0, st>>>(partials, chunks, max_norm, sum_out, norm_out,
                                                   grad_mul_out, nullptr, nonfinite_out);
    return check_launch("hbt_grad_norm_noalloc");
}

int32_t hbt_scale_inplace(void* const* tensors, const int64_t* numels, int32_t count,
                          int32_t dtype, float unscale, const float* grad_mul, void* stream) {
    clear_error();
    if (count < 0 || count > kMaxT || (count > 0 && (tensors == nullptr || numels == nullptr))) {
        set_error("hbt_scale_inplace: bad table (count=%d)", count);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if (dtype != F32 && dtype != BF16 && dtype != F16) {
        set_error("hbt_scale_inplace: dtype %d is not F32, BF16 or F16 (float64: hbt_scale_inplace_f64)", dtype);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    ScaleTable tab{};
    tab.count = count;
    const int64_t tile = dtype == F32 ? scale_tile<F32>() : scale_tile<BF16>();
    int64_t blocks = 0;
    for (int i = 0; i < count; ++i) {
        if (numels[i] < 0 || (numels[i] > 0 && tensors[i] == nullptr)) {
            set_error("hbt_scale_inplace: tensor %d has a bad pointer or numel", i);
            return HBT_ERR_INVALID_ARGUMENT;
        }
        tab.x[i] = tensors[i];
        tab.n[i] = numels[i];
        tab.vec_ok[i] = aligned(tensors[i], 16);
        tab.first_block[i] = blocks;
        blocks += (numels[i] + tile - 1) / tile;
    }
    tab.first_block[count] = blocks;
    for (int i = count + 1; i <= kMaxT; ++i) tab.first_block[i] = blocks;
    hipStream_t st = as_stream(stream);
    const int threads = dtype == F32 ? scale_block<F32>() : scale_block<BF16>();
    return launch_sliced("hbt_scale_inplace", blocks, threads, [&](int64_t first, dim3 grid) {
        if (dtype == F32) scale_kernel<F32><<<grid, threads, 0, st>>>(tab, unscale, grad_mul, first);
        else if (dtype == BF16) scale_kernel<BF16><<<grid, threads, 0, st>>>(tab, unscale, grad_mul, first);
        else scale_kernel<F16><<<grid, threads, 0, st>>>(tab, unscale, grad_mul, first);
    });
}

int32_t hbt_grad_accumulate(void* const* accumulators, const void* const* grads, const int64_t* numels,
                            int32_t count, int32_t acc_dtype, int32_t grad_dtype, int32_t flags, void* stream) {
    clear_error();
    if (count < 0 || count > kMaxT ||
        (count > 0 && (accumulators == nullptr || grads == nullptr || numels == nullptr))) {
        set_error("hbt_grad_accumulate: bad table (count=%d)", count);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    const auto float_code = [](int32_t d) { return d == F32 || d == BF16 || d == F16; };
    const bool f64 = acc_dtype == HBT_DTYPE_F64;
    if (!(float_code(acc_dtype) || f64) || !(float_code(grad_dtype) || (f64 && grad_dtype == HBT_DTYPE_F64))) {
        set_error("hbt_grad_accumulate: dtypes (accumulator %d, gradient %d) must be F32, BF16 or F16 "
                  "(or an F64 accumulator, whose gradient may also be F64)",
                  acc_dtype, grad_dtype);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if ((flags & ~HBT_ACCUMULATE_ASSIGN) != 0) {
        set_error("hbt_grad_accumulate: unknown flags 0x%x", static_cast<unsigned>(flags));
        return HBT_ERR_INVALID_ARGUMENT;
    }
    const uintptr_t acc_bytes = static_cast<uintptr_t>(dtype_size(acc_dtype));
    const uintptr_t grad_bytes = static_cast<uintptr_t>(dtype_size(grad_dtype));
    AccumTable tab{};
    tab.count = count;
    int64_t blocks = 0;
    for (int i = 0; i < count; ++i) {
        if (numels[i] < 0 || (numels[i] > 0 && (accumulators[i] == nullptr || grads[i] == nullptr))) {
            set_error("hbt_grad_accumulate: pair %d has a bad pointer or numel", i);
            return HBT_ERR_INVALID_ARGUMENT;
        }
        tab.acc[i] = accumulators[i];
        tab.grad[i] = grads[i];
        tab.n[i] = numels[i];
        tab.vec_ok[i] = aligned(accumulators[i], 4 * acc_bytes) && aligned(grads[i], 4 * grad_bytes);
        tab.first_block[i] = blocks;
        blocks += (numels[i] + kAccumTile - 1) / kAccumTile;
    }
    tab.first_block[count] = blocks;
    for (int i = count + 1; i <= kMaxT; ++i) tab.first_block[i] = blocks;
    hipStream_t st = as_stream(stream);
    const bool assign = (flags & HBT_ACCUMULATE_ASSIGN) != 0;
    return launch_sliced("hbt_grad_accumulate", blocks, kAccumBlock, [&](int64_t first, dim3 grid) {
#define HBT_ACC(GD, AD)                                                                        \
    do {                                                                                       \
        if (assign) accumulate_kernel<GD, AD, true><<<grid, kAccumBlock, 0, st>>>(tab, first); \
        else accumulate_kernel<GD, AD, false><<<grid, kAccumBlock, 0, st>>>(tab, first);       \
    } while (0)
#define HBT_ACC_A(GD)                                  \
    do {                                               \
        if (acc_dtype == F32) HBT_ACC(GD, F32);        \
        else if (acc_dtype == BF16) HBT_ACC(GD, BF16); \
        else HBT_ACC(GD, F16);                         \
    } while (0)
#define HBT_ACC64(SB, SH)                                                                          \
    do {                                                                                           \
        if (assign) accumulate_f64_kernel<SB, SH, true><<<grid, kAccumBlock, 0, st>>>(tab, first); \
        else accumulate_f64_kernel<SB, SH, false><<<grid, kAccumBlock, 0, st>>>(tab, first);       \
    } while (0)
        if (f64) {
            if (grad_dtype == HBT_DTYPE_F64) HBT_ACC64(8, false);
            else if (grad_dtype == F32) HBT_ACC64(4, false);
            else if (grad_dtype == BF16) HBT_ACC64(2, false);
            else HBT_ACC64(2, true);
        } else if (grad_dtype == F32) {
            HBT_ACC_A(F32);
        } else if (grad_dtype == BF16) {
            HBT_ACC_A(BF16);
        } else {
            HBT_ACC_A(F16);
        }
#undef HBT_ACC_A
#undef HBT_ACC64
#undef HBT_ACC
    });
}

int32_t hbt_grad_local_share(const void* const* rank_grads, int32_t group_size, int32_t rank,
                             int64_t shard_numel, int64_t valid_numel, int32_t in_dtype,
                             int32_t reduce_dtype, float divisor, int32_t out_dtype, void* out, void* stream) {
    clear_error();
    return local_share("hbt_grad_local_share", rank_grads, group_size, rank, shard_numel, valid_numel, in_dtype,
                       reduce_dtype, divisor, out_dtype, out, nullptr, nullptr, as_stream(stream));
}

int32_t hbt_grad_local_share_sqnorm(const void* const* rank_grads, int32_t group_size, int32_t rank,
                                    int64_t shard_numel, int64_t valid_numel, int32_t in_dtype,
                                    int32_t reduce_dtype, float divisor, int32_t out_dtype, void* out,
                                    double* partials, double* tile_scratch, void* stream) {
    clear_error();
    if (partials == nullptr || tile_scratch == nullptr) {
        set_error("hbt_grad_local_share_sqnorm: null partials or tile scratch");
        return HBT_ERR_INVALID_ARGUMENT;
    }
    return local_share("hbt_grad_local_share_sqnorm", rank_grads, group_size, rank, shard_numel, valid_numel,
                       in_dtype, reduce_dtype, divisor, out_dtype, out, partials, tile_scratch, as_stream(stream));
}

int32_t hbt_grad_local_share_accumulated(const void* const* rank_grads, const void* const* accumulators,
                                         int32_t group_size, int32_t rank, int64_t shard_numel, int64_t valid_numel,
                                         int32_t in_dtype, int32_t reduce_dtype, float divisor, int32_t out_dtype,
                                         void* out, double* partials, double* tile_scratch, void* stream) {
    clear_error();
    if (accumulators == nullptr) {
        set_error("hbt_grad_local_share_accumulated: null accumulator table");
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if ((partials == nullptr) != (tile_scratch == nullptr)) {
        set_error("hbt_grad_local_share_accumulated: partials and tile scratch must both be given or both null");
        return HBT_ERR_INVALID_ARGUMENT;
    }
    return local_share("hbt_grad_local_share_accumulated", rank_grads, group_size, rank, shard_numel, valid_numel,
                       in_dtype, reduce_dtype, divisor, out_dtype, out, partials, tile_scratch, as_stream(stream),
                       accumulators);
}

static int32_t sgd_step_impl(const char* who, void* const* params, void* const* grads, void* const* momentum_buffers,
                     const int64_t* numels, int32_t count, int32_t param_dtype, int32_t grad_dtype, float unscale,
                     const float* grad_mul, float weight_decay, float momentum, float one_minus_dampening,
                     float neg_lr, const SgdScalars* slot, int32_t flags, void* stream) {
    clear_error();
    if (count < 0 || count > kMaxT) {
        set_error("%s: count must lie in [0, %d], got %d", who, kMaxT, count);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if (!optimizer_dtypes_ok(param_dtype, grad_dtype)) {
        set_error("%s: (parameter, gradient) dtypes (%d, %d) are not (F32, F32), (F32, BF16), "
                  "(BF16, BF16) or (F16, F16)", who, param_dtype, grad_dtype);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    const int32_t known = HBT_SGD_MOMENTUM | HBT_SGD_FIRST_STEP | HBT_SGD_NESTEROV | HBT_SGD_WEIGHT_DECAY |
                          HBT_STEP_WRITE_GRAD;
    if ((flags & ~known) != 0 ||
        ((flags & (HBT_SGD_FIRST_STEP | HBT_SGD_NESTEROV)) != 0 && (flags & HBT_SGD_MOMENTUM) == 0)) {
        set_error("%s: bad flags 0x%x", who, flags);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    const bool with_momentum = (flags & HBT_SGD_MOMENTUM) != 0;
    if (count > 0 && (params == nullptr || grads == nullptr || numels == nullptr ||
                      (with_momentum && momentum_buffers == nullptr))) {
        set_error("%s: null pointer argument", who);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    SgdTable tab{};
    tab.count = count;
    const bool write_back = (flags & HBT_STEP_WRITE_GRAD) != 0;
    const int64_t tile = adam_tile_of(param_dtype, write_back);
    const int vec = param_dtype == F32 ? adam_vec<F32>() : adam_vec<BF16>();
    const uintptr_t state_align = static_cast<uintptr_t>(vec * dtype_size(param_dtype));
    const uintptr_t grad_align = static_cast<uintptr_t>(vec * dtype_size(grad_dtype));
    int64_t blocks = 0;
    for (int i = 0; i < count; ++i) {
        if (numels[i] < 0 || (numels[i] > 0 && (params[i] == nullptr || grads[i] == nullptr ||
                                                (with_momentum && momentum_buffers[i] == nullptr)))) {
            set_error("%s: tensor %d has a bad pointer or numel", who, i);
            return HBT_ERR_INVALID_ARGUMENT;
        }
        tab.p[i] = params[i];
        tab.g[i] = grads[i];
        tab.buf[i] = with_momentum ? momentum_buffers[i] : nullptr;
        tab.n[i] = numels[i];
        tab.vec_ok[i] = aligned(params[i], state_align) && aligned(grads[i], grad_align) &&
                        (!with_momentum || aligned(momentum_buffers[i], state_align));
        tab.first_block[i] = blocks;
        blocks += (numels[i] + tile - 1) / tile;
    }
    tab.first_block[count] = blocks;
    for (int i = count + 1; i <= kMaxT; ++i) tab.first_block[i] = blocks;
    const SgdScalars sc = sgd_scalars(param_dtype, unscale, weight_decay, momentum, one_minus_dampening, neg_lr,
                                      flags);
    const int mode = !with_momentum ? kSgdPlain : ((flags & HBT_SGD_FIRST_STEP) ? kSgdFirst : kSgdMomentum);
    const bool scaled = unscale != 1.0f;
    hipStream_t st = as_stream(stream);
    return launch_sliced(who, blocks, kAdamBlock, [&](int64_t first, dim3 grid) {
#define HBT_SGD(PD, GD, SCALED, MODE, WB) \
    sgd_kernel<PD, GD, SCALED, MODE, WB><<<grid, kAdamBlock, 0, st>>>(tab, sc, slot, grad_mul, first)
#define HBT_SGD_WB(PD, GD, SCALED, MODE)                     \
    do {                                                     \
        if (write_back) HBT_SGD(PD, GD, SCALED, MODE, true); \
        else HBT_SGD(PD, GD, SCALED, MODE, false);           \
    } while (0)
#define HBT_SGD_MODES(PD, GD, SCALED)                                      \
    do {                                                                   \
        if (mode == kSgdPlain) HBT_SGD_WB(PD, GD, SCALED, kSgdPlain);      \
        else if (mode == kSgdFirst) HBT_SGD_WB(PD, GD, SCALED, kSgdFirst); \
        else HBT_SGD_WB(PD, GD, SCALED, kSgdMomentum);                     \
    } while (0)
#define HBT_SGD_SCALED(PD, GD)                   \
    do {                                         \
        if (scaled) HBT_SGD_MODES(PD, GD, true); \
        else HBT_SGD_MODES(PD, GD, false);       \
    } while (0)
        if (param_dtype == F32 && grad_dtype == F32) HBT_SGD_SCALED(F32, F32);
        else if (param_dtype == F32) HBT_SGD_SCALED(F32, BF16);
        else if (param_dtype == BF16) HBT_SGD_SCALED(BF16, BF16);
        else HBT_SGD_SCALED(F16, F16);
#undef HBT_SGD_SCALED
#undef HBT_SGD_MODES
#undef HBT_SGD_WB
#undef HBT_SGD
    });
}

static int32_t adamw_step_f64_impl(const char* who, double* const* params, double* const* grads, double* const* exp_avgs,
                           double* const* exp_avg_sqs, const int64_t* numels, int32_t count, double unscale,
                           const double* grad_mul, double decay, double lerp_weight, double beta2,
                           double one_minus_beta2, double bias_correction2_sqrt, double eps, double neg_step_size,
                           const AdamScalarsF64* slot, int32_t flags, void* stream) {
    clear_error();
    if (count < 0 || count > kMaxT) {
        set_error("%s: count must lie in [0, %d], got %d", who, kMaxT, count);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if ((flags & ~HBT_STEP_WRITE_GRAD) != 0) {
        set_error("%s: unknown flags 0x%x", who, static_cast<unsigned>(flags));
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if (count > 0 && (params == nullptr || grads == nullptr || exp_avgs == nullptr || exp_avg_sqs == nullptr ||
                      numels == nullptr)) {
        set_error("%s: null table pointer", who);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    const bool write_back = (flags & HBT_STEP_WRITE_GRAD) != 0;
    const int64_t tile = write_back ? adam_f64_tile<true>() : adam_f64_tile<false>();
    AdamTable tab{};
    tab.count = count;
    int64_t blocks = 0;
    for (int i = 0; i < count; ++i) {
        if (numels[i] < 0 || (numels[i] > 0 && (params[i] == nullptr || grads[i] == nullptr ||
                                                exp_avgs[i] == nullptr || exp_avg_sqs[i] == nullptr))) {
            set_error("%s: tensor %d has a bad pointer or numel", who, i);
            return HBT_ERR_INVALID_ARGUMENT;
        }
        tab.p[i] = params[i];
        tab.g[i] = grads[i];
        tab.m[i] = exp_avgs[i];
        tab.v[i] = exp_avg_sqs[i];
        tab.n[i] = numels[i];
        tab.vec_ok[i] = aligned(params[i], 16) && aligned(grads[i], 16) && aligned(exp_avgs[i], 16) &&
                        aligned(exp_avg_sqs[i], 16);
        tab.first_block[i] = blocks;
        blocks += (numels[i] + tile - 1) / tile;
    }
    tab.first_block[count] = blocks;
    for (int i = count + 1; i <= kMaxT; ++i) tab.first_block[i] = blocks;
    const AdamScalarsF64 s = adam_scalars_f64(unscale, decay, lerp_weight, beta2, one_minus_beta2,
                                              bias_correction2_sqrt, eps, neg_step_size);
    const bool lerp_small = std::fabs(lerp_weight) < 0.5;
    const bool scaled = unscale != 1.0;
    hipStream_t st = as_stream(stream);
    return launch_sliced(who, blocks, kAdamBlock, [&](int64_t first, dim3 grid) {
#define HBT_ADAMW64(SMALL, SCALED, WB) \
    adamw_f64_kernel<SMALL, SCALED, WB><<<grid, kAdamBlock, 0, st>>>(tab, s, slot, grad_mul, first)
#define HBT_ADAMW64_WB(SMALL, SCALED)                     \
    do {                                                  \
        if (write_back) HBT_ADAMW64(SMALL, SCALED, true); \
        else HBT_ADAMW64(SMALL, SCALED, false);           \
    } while (0)
#define HBT_ADAMW64_SCALED(SMALL)                \
    do {                                         \
        if (scaled) HBT_ADAMW64_WB(SMALL, true); \
        else HBT_ADAMW64_WB(SMALL, false);       \
    } while (0)
        if (lerp_small) HBT_ADAMW64_SCALED(true);
        else HBT_ADAMW64_SCALED(false);
#undef HBT_ADAMW64_SCALED
#undef HBT_ADAMW64_WB
#undef HBT_ADAMW64
    });
}

static int32_t sgd_step_f64_impl(const char* who, double* const* params, double* const* grads, double* const* momentum_buffers,
                         const int64_t* numels, int32_t count, double unscale, const double* grad_mul,
                         double weight_decay, double momentum, double one_minus_dampening, double neg_lr,
                         const SgdScalarsF64* slot, int32_t flags, void* stream) {
    clear_error();
    if (count < 0 || count > kMaxT) {
        set_error("%s: count must lie in [0, %d], got %d", who, kMaxT, count);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    const int32_t known = HBT_SGD_MOMENTUM | HBT_SGD_FIRST_STEP | HBT_SGD_NESTEROV | HBT_SGD_WEIGHT_DECAY |
                          HBT_STEP_WRITE_GRAD;
    if ((flags & ~known) != 0 ||
        ((flags & (HBT_SGD_FIRST_STEP | HBT_SGD_NESTEROV)) != 0 && (flags & HBT_SGD_MOMENTUM) == 0)) {
        set_error("%s: bad flags 0x%x", who, flags);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    const bool with_momentum = (flags & HBT_SGD_MOMENTUM) != 0;
    if (count > 0 && (params == nullptr || grads == nullptr || numels == nullptr ||
                      (with_momentum && momentum_buffers == nullptr))) {
        set_error("%s: null pointer argument", who);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    const bool write_back = (flags & HBT_STEP_WRITE_GRAD) != 0;
    const int64_t tile = write_back ? adam_f64_tile<true>() : adam_f64_tile<false>();
    SgdTable tab{};
    tab.count = count;
    int64_t blocks = 0;
    for (int i = 0; i < count; ++i) {
        if (numels[i] < 0 || (numels[i] > 0 && (params[i] == nullptr || grads[i] == nullptr ||
                                                (with_momentum && momentum_buffers[i] == nullptr)))) {
            set_error("%s: tensor %d has a bad pointer or numel", who, i);
            return HBT_ERR_INVALID_ARGUMENT;
        }
        tab.p[i] = params[i];
        tab.g[i] = grads[i];
        tab.buf[i] = with_momentum ? momentum_buffers[i] : nullptr;
        tab.n[i] = numels[i];
        tab.vec_ok[i] = aligned(params[i], 16) && aligned(grads[i], 16) &&
                        (!with_momentum || aligned(momentum_buffers[i], 16));
        tab.first_block[i] = blocks;
        blocks += (numels[i] + tile - 1) / tile;
    }
    tab.first_block[count] = blocks;
    for (int i = count + 1; i <= kMaxT; ++i) tab.first_block[i] = blocks;
    const SgdScalarsF64 sc = sgd_scalars_f64(unscale, weight_decay, momentum, one_minus_dampening, neg_lr, flags);
    const int mode = !with_momentum ? kSgdPlain : ((flags & HBT_SGD_FIRST_STEP) ? kSgdFirst : kSgdMomentum);
    const bool scaled = unscale != 1.0;
    hipStream_t st = as_stream(stream);
    return launch_sliced(who, blocks, kAdamBlock, [&](int64_t first, dim3 grid) {
#define HBT_SGD64(SCALED, MODE, WB) sgd_f64_kernel<SCALED, MODE, WB><<<grid, kAdamBlock, 0, st>>>(tab, sc, slot, grad_mul, first)
#define HBT_SGD64_WB(SCALED, MODE)                     \
    do {                                               \
        if (write_back) HBT_SGD64(SCALED, MODE, true); \
        else HBT_SGD64(SCALED, MODE, false);           \
    } while (0)
#define HBT_SGD64_MODES(SCALED)                                      \
    do {                                                             \
        if (mode == kSgdPlain) HBT_SGD64_WB(SCALED, kSgdPlain);      \
        else if (mode == kSgdFirst) HBT_SGD64_WB(SCALED, kSgdFirst); \
        else HBT_SGD64_WB(SCALED, kSgdMomentum);                     \
    } while (0)
        if (scaled) HBT_SGD64_MODES(true);
        else HBT_SGD64_MODES(false);
#undef HBT_SGD64_MODES
#undef HBT_SGD64_WB
#undef HBT_SGD64
    });
}

int32_t hbt_scale_inplace_f64(double* const* tensors, const int64_t* numels, int32_t count, double unscale,
                              const double* grad_mul, void* stream) {
    clear_error();
    if (count < 0 || count > kMaxT || (count > 0 && (tensors == nullptr || numels == nullptr))) {
        set_error("hbt_scale_inplace_f64: bad table (count=%d)", count);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    ScaleTable tab{};
    tab.count = count;
    int64_t blocks = 0;
    for (int i = 0; i < count; ++i) {
        if (numels[i] < 0 || (numels[i] > 0 && tensors[i] == nullptr)) {
            set_error("hbt_scale_inplace_f64: tensor %d has a bad pointer or numel", i);
            return HBT_ERR_INVALID_ARGUMENT;
        }
        tab.x[i] = tensors[i];
        tab.n[i] = numels[i];
        tab.vec_ok[i] = aligned(tensors[i], 16);
        tab.first_block[i] = blocks;
        blocks += (numels[i] + kScaleF64Tile - 1) / kScaleF64Tile;
    }
    tab.first_block[count] = blocks;
    for (int i = count + 1; i <= kMaxT; ++i) tab.first_block[i] = blocks;
    hipStream_t st = as_stream(stream);
    return launch_sliced("hbt_scale_inplace_f64", blocks, 32, [&](int64_t first, dim3 grid) {
        scale_f64_kernel<<<grid, 32, 0, st>>>(tab, unscale, grad_mul, first);
    });
}

// ---- the eager steps and their slot forms ---------------------------------------------
int32_t hbt_adamw_step(void* const* params, void* const* grads, void* const* exp_avgs,
                       void* const* exp_avg_sqs, const int64_t* numels, int32_t count,
                       int32_t param_dtype, int32_t grad_dtype, float unscale, const float* grad_mul,
                       float decay, float lerp_weight, float beta2, float one_minus_beta2,
                       float bias_correction2_sqrt, float eps, float neg_step_size, int32_t flags,
                       void* stream) {
    return adamw_step_impl("hbt_adamw_step", params, grads, exp_avgs, exp_avg_sqs, numels, count, param_dtype,
                           grad_dtype, unscale, grad_mul, decay, lerp_weight, beta2, one_minus_beta2,
                           bias_correction2_sqrt, eps, neg_step_size, nullptr, flags, stream);
}

int32_t hbt_adamw_step_slot(void* const* params, void* const* grads, void* const* exp_avgs,
                            void* const* exp_avg_sqs, const int64_t* numels, int32_t count,
                            int32_t param_dtype, int32_t grad_dtype, float unscale, const float* grad_mul,
                            float decay, float lerp_weight, float beta2, float one_minus_beta2,
                            float bias_correction2_sqrt, float eps, float neg_step_size, const void* slot,
                            int32_t flags, void* stream) {
    clear_error();
    if (!slot_ok("hbt_adamw_step_slot", slot)) return HBT_ERR_INVALID_ARGUMENT;
    return adamw_step_impl("hbt_adamw_step_slot", params, grads, exp_avgs, exp_avg_sqs, numels, count, param_dtype,
                           grad_dtype, unscale, grad_mul, decay, lerp_weight, beta2, one_minus_beta2,
                           bias_correction2_sqrt, eps, neg_step_size, static_cast<const AdamScalars*>(slot), flags,
                           stream);
}

int32_t hbt_adamw_write_scalars(void* slot, int32_t param_dtype, float unscale, float decay, float lerp_weight,
                                float beta2, float one_minus_beta2, float bias_correction2_sqrt, float eps,
                                float neg_step_size, void* stream) {
    clear_error();
    if (param_dtype != F32 && param_dtype != BF16 && param_dtype != F16) {
        set_error("hbt_adamw_write_scalars: param_dtype %d is not F32, BF16 or F16", param_dtype);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    return write_slot("hbt_adamw_write_scalars", slot,
                      adam_scalars(param_dtype, unscale, decay, lerp_weight, beta2, one_minus_beta2,
                                   bias_correction2_sqrt, eps, neg_step_size),
                      as_stream(stream));
}

int32_t hbt_sgd_step(void* const* params, void* const* grads, void* const* momentum_buffers,
                     const int64_t* numels, int32_t count, int32_t param_dtype, int32_t grad_dtype, float unscale,
                     const float* grad_mul, float weight_decay, float momentum, float one_minus_dampening,
                     float neg_lr, int32_t flags, void* stream) {
    return sgd_step_impl("hbt_sgd_step", params, grads, momentum_buffers, numels, count, param_dtype, grad_dtype,
                         unscale, grad_mul, weight_decay, momentum, one_minus_dampening, neg_lr, nullptr, flags,
                         stream);
}

int32_t hbt_sgd_step_slot(void* const* params, void* const* grads, void* const* momentum_buffers,
                          const int64_t* numels, int32_t count, int32_t param_dtype, int32_t grad_dtype,
                          float unscale, const float* grad_mul, float weight_decay, float momentum,
                          float one_minus_dampening, float neg_lr, const void* slot, int32_t flags, void* stream) {
    clear_error();
    if (!slot_ok("hbt_sgd_step_slot", slot)) return HBT_ERR_INVALID_ARGUMENT;
    return sgd_step_impl("hbt_sgd_step_slot", params, grads, momentum_buffers, numels, count, param_dtype,
                         grad_dtype, unscale, grad_mul, weight_decay, momentum, one_minus_dampening, neg_lr,
                         static_cast<const SgdScalars*>(slot), flags, stream);
}

int32_t hbt_sgd_write_scalars(void* slot, int32_t param_dtype, float unscale, float weight_decay, float momentum,
                              float one_minus_dampening, float neg_lr, int32_t flags, void* stream) {
    clear_error();
    if (param_dtype != F32 && param_dtype != BF16 && param_dtype != F16) {
        set_error("hbt_sgd_write_scalars: param_dtype %d is not F32, BF16 or F16", param_dtype);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if (!sgd_flags_ok("hbt_sgd_write_scalars", flags)) return HBT_ERR_INVALID_ARGUMENT;
    return write_slot("hbt_sgd_write_scalars", slot,
                      sgd_scalars(param_dtype, unscale, weight_decay, momentum, one_minus_dampening, neg_lr, flags),
                      as_stream(stream));
}

int32_t hbt_adamw_step_f64(double* const* params, double* const* grads, double* const* exp_avgs,
                           double* const* exp_avg_sqs, const int64_t* numels, int32_t count, double unscale,
                           const double* grad_mul, double decay, double lerp_weight, double beta2,
                           double one_minus_beta2, double bias_correction2_sqrt, double eps, double neg_step_size,
                           int32_t flags, void* stream) {
    return adamw_step_f64_impl("hbt_adamw_step_f64", params, grads, exp_avgs, exp_avg_sqs, numels, count, unscale,
                               grad_mul, decay, lerp_weight, beta2, one_minus_beta2, bias_correction2_sqrt, eps,
                               neg_step_size, nullptr, flags, stream);
}

int32_t hbt_adamw_step_f64_slot(double* const* params, double* const* grads, double* const* exp_avgs,
                                double* const* exp_avg_sqs, const int64_t* numels, int32_t count, double unscale,
                                const double* grad_mul, double decay, double lerp_weight, double beta2,
                                double one_minus_beta2, double bias_correction2_sqrt, double eps,
                                double neg_step_size, const void* slot, int32_t flags, void* stream) {
    clear_error();
    if (!slot_ok("hbt_adamw_step_f64_slot", slot)) return HBT_ERR_INVALID_ARGUMENT;
    return adamw_step_f64_impl("hbt_adamw_step_f64_slot", params, grads, exp_avgs, exp_avg_sqs, numels, count,
                               unscale, grad_mul, decay, lerp_weight, beta2, one_minus_beta2, bias_correction2_sqrt,
                               eps, neg_step_size, static_cast<const AdamScalarsF64*>(slot), flags, stream);
}

int32_t hbt_adamw_write_scalars_f64(void* slot, double unscale, double decay, double lerp_weight, double beta2,
                                    double one_minus_beta2, double bias_correction2_sqrt, double eps,
                                    double neg_step_size, void* stream) {
    clear_error();
    return write_slot("hbt_adamw_write_scalars_f64", slot,
                      adam_scalars_f64(unscale, decay, lerp_weight, beta2, one_minus_beta2, bias_correction2_sqrt,
                                       eps, neg_step_size),
                      as_stream(stream));
}

int32_t hbt_sgd_step_f64(double* const* params, double* const* grads, double* const* momentum_buffers,
                         const int64_t* numels, int32_t count, double unscale, const double* grad_mul,
                         double weight_decay, double momentum, double one_minus_dampening, double neg_lr,
                         int32_t flags, void* stream) {
    return sgd_step_f64_impl("hbt_sgd_step_f64", params, grads, momentum_buffers, numels, count, unscale, grad_mul,
                             weight_decay, momentum, one_minus_dampening, neg_lr, nullptr, flags, stream);
}

int32_t hbt_sgd_step_f64_slot(double* const* params, double* const* grads, double* const* momentum_buffers,
                              const int64_t* numels, int32_t count, double unscale, const double* grad_mul,
                              double weight_decay, double momentum, double one_minus_dampening, double neg_lr,
                              const void* slot, int32_t flags, void* stream) {
    clear_error();
    if (!slot_ok("hbt_sgd_step_f64_slot", slot)) return HBT_ERR_INVALID_ARGUMENT;
    return sgd_step_f64_impl("hbt_sgd_step_f64_slot", params, grads, momentum_buffers, numels, count, unscale,
                             grad_mul, weight_decay, momentum, one_minus_dampening, neg_lr,
                             static_cast<const SgdScalarsF64*>(slot), flags, stream);
}

int32_t hbt_sgd_write_scalars_f64(void* slot, double unscale, double weight_decay, double momentum,
                                  double one_minus_dampening, double neg_lr, int32_t flags, void* stream) {
    clear_error();
    if (!sgd_flags_ok("hbt_sgd_write_scalars_f64", flags)) return HBT_ERR_INVALID_ARGUMENT;
    return write_slot("hbt_sgd_write_scalars_f64", slot,
                      sgd_scalars_f64(unscale, weight_decay, momentum, one_minus_dampening, neg_lr, flags),
                      as_stream(stream));
}

int32_t hbt_adamw_scalar_record(void* record, int32_t param_dtype, float unscale, float decay, float lerp_weight,
                                float beta2, float one_minus_beta2, float bias_correction2_sqrt, float eps,
                                float neg_step_size) {
    clear_error();
    if (param_dtype != F32 && param_dtype != BF16 && param_dtype != F16) {
        set_error("hbt_adamw_scalar_record: param_dtype %d is not F32, BF16 or F16", param_dtype);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    return format_slot("hbt_adamw_scalar_record", record,
                       adam_scalars(param_dtype, unscale, decay, lerp_weight, beta2, one_minus_beta2,
                                    bias_correction2_sqrt, eps, neg_step_size));
}

int32_t hbt_sgd_scalar_record(void* record, int32_t param_dtype, float unscale, float weight_decay, float momentum,
                              float one_minus_dampening, float neg_lr, int32_t flags) {
    clear_error();
    if (param_dtype != F32 && param_dtype != BF16 && param_dtype != F16) {
        set_error("hbt_sgd_scalar_record: param_dtype %d is not F32, BF16 or F16", param_dtype);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if (!sgd_flags_ok("hbt_sgd_scalar_record", flags)) return HBT_ERR_INVALID_ARGUMENT;
    return format_slot("hbt_sgd_scalar_record", record,
                       sgd_scalars(param_dtype, unscale, weight_decay, momentum, one_minus_dampening, neg_lr, flags));
}

int32_t hbt_adamw_scalar_record_f64(void* record, double unscale, double decay, double lerp_weight, double beta2,
                                    double one_minus_beta2, double bias_correction2_sqrt, double eps,
                                    double neg_step_size) {
    clear_error();
    return format_slot("hbt_adamw_scalar_record_f64", record,
                       adam_scalars_f64(unscale, decay, lerp_weight, beta2, one_minus_beta2, bias_correction2_sqrt,
                                        eps, neg_step_size));
}

int32_t hbt_sgd_scalar_record_f64(void* record, double unscale, double weight_decay, double momentum,
                                  double one_minus_dampening, double neg_lr, int32_t flags) {
    clear_error();
    if (!sgd_flags_ok("hbt_sgd_scalar_record_f64", flags)) return HBT_ERR_INVALID_ARGUMENT;
    return format_slot("hbt_sgd_scalar_record_f64", record,
                       sgd_scalars_f64(unscale, weight_decay, momentum, one_minus_dampening, neg_lr, flags));
}

int32_t hbt_write_words(void* dst, const uint32_t* words, int64_t count, void* stream) {
    clear_error();
    return write_words("hbt_write_words", dst, words, count, as_stream(stream));
}

}  // extern "C"
