// Fused clip + AdamW step and the deterministic fp64 gradient norm (gfx950).
//
// Both kernels stream their operands exactly once from HBM with 16-byte
// non-temporal loads and stores.  Work is split into fixed-size tiles; a launch
// covers a table of up to HBT_MAX_TENSORS_PER_LAUNCH tensors, so a list of flat
// shards (or of DDP-style per-parameter tensors) costs one launch per 16 tensors.
#include <cmath>
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

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// AdamW (and SGD): 32-thread workgroups, i.e. half a wavefront each, two 16-byte
// vectors per lane and operand, 256 elements per workgroup.  Measured on MI355X on
// this 4-read/3-write stream (1e9 elements): 6.38 TB/s, against 5.87 TB/s for
// full-wave 64-thread workgroups, 5.4 TB/s for 128 threads and under 5 TB/s for
// 16 threads or 256-thread workgroups; persistent grid-stride variants are slower.
#ifndef HBT_ADAM_BLOCK
#define HBT_ADAM_BLOCK 32
#endif
constexpr int kAdamBlock = HBT_ADAM_BLOCK;
constexpr int kAdamUnroll = 2;
constexpr int64_t kAdamTile = int64_t(kAdamBlock) * 4 * kAdamUnroll;

// Norm: 1024-thread workgroups, each summing one contiguous chunk of 8 tiles; a tile
// is one 16-byte load per lane (4 fp32 or 8 bf16 gradients).
constexpr int kNormBlock = 1024;
constexpr int kNormTilesPerChunk = 8;
template <typename GradT>
constexpr int64_t norm_tile() { return int64_t(kNormBlock) * (16 / sizeof(GradT)); }
template <typename GradT>
constexpr int64_t norm_chunk() { return norm_tile<GradT>() * kNormTilesPerChunk; }

// ---- 16-byte memory helpers ------------------------------------------------------
// Every operand is touched exactly once per step, so loads and stores are marked
// non-temporal: the lines are not kept in L2/MALL for reuse that never comes.
__device__ __forceinline__ f32x4 ld4_nt(const float* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
}
__device__ __forceinline__ void st4_nt(float* p, f32x4 x) {
    __builtin_nontemporal_store(x, reinterpret_cast<f32x4*>(p));
}
// Four gradient values widened to fp32 (bf16 widening is exact).
__device__ __forceinline__ f32x4 ld_grad4_nt(const float* p) { return ld4_nt(p); }
__device__ __forceinline__ f32x4 ld_grad4_nt(const uint16_t* p) {
    const u32x2 w = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
    return f32x4{bf16_to_f32(w.x & 0xFFFFu), bf16_to_f32(w.x >> 16), bf16_to_f32(w.y & 0xFFFFu),
                 bf16_to_f32(w.y >> 16)};
}
// Eight bf16 gradients (one 16-byte load) widened to fp32, as two 4-vectors.
__device__ __forceinline__ void ld_bf16x8_nt(const uint16_t* p, f32x4& lo, f32x4& hi) {
    typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
    const u32x4v w = __builtin_nontemporal_load(reinterpret_cast<const u32x4v*>(p));
    lo = f32x4{bf16_to_f32(w.x & 0xFFFFu), bf16_to_f32(w.x >> 16), bf16_to_f32(w.y & 0xFFFFu),
               bf16_to_f32(w.y >> 16)};
    hi = f32x4{bf16_to_f32(w.z & 0xFFFFu), bf16_to_f32(w.z >> 16), bf16_to_f32(w.w & 0xFFFFu),
               bf16_to_f32(w.w >> 16)};
}
__device__ __forceinline__ float ld_grad1(const float* p) { return *p; }
__device__ __forceinline__ float ld_grad1(const uint16_t* p) { return bf16_to_f32(*p); }

// Wait for every outstanding vector-memory load of this wave (s_waitcnt vmcnt(0)).
// Issuing a lane's four operand streams one after the other, rather than all at
// once, keeps the HBM request mix per wave simpler and measured ~2% faster.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// ---- AdamW -----------------------------------------------------------------------
struct AdamTable {
    float* p[kMaxT];
    const void* g[kMaxT];
    float* m[kMaxT];
    float* v[kMaxT];
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
    float eps;
    float neg_step;
};

// One element of torch's single-tensor AdamW, preceded by the unscale and clip
// multiplies.  Compiled with -ffp-contract=off: only the two explicit fmaf calls fuse.
template <bool kLerpSmall, bool kUnscale>
__device__ __forceinline__ void adamw_update(float& p, float g, float& m, float& v, float gmul,
                                             const AdamScalars& s) {
    if constexpr (kUnscale) g = g * s.unscale;
    g = g * gmul;
    p = p * s.decay;
    const float diff = g - m;
    if constexpr (kLerpSmall) {
        m = __builtin_fmaf(s.lerp_w, diff, m);
    } else {
        m = __builtin_fmaf(s.lerp_w_minus_1, diff, g);
    }
    v = v * s.beta2;
    v = __builtin_fmaf(s.one_minus_beta2 * g, g, v);
    const float denom = __builtin_sqrtf(v) / s.bc2_sqrt + s.eps;
    p = p + (s.neg_step * m) / denom;
}

template <typename GradT, bool kLerpSmall, bool kUnscale>
__global__ __launch_bounds__(kAdamBlock) void adamw_kernel(AdamTable tab, AdamScalars s,
                                                           const float* __restrict__ grad_mul) {
    const int64_t block = blockIdx.x;
    int t = 0;
    while (t + 1 < tab.count && block >= tab.first_block[t + 1]) ++t;
    const int64_t base = (block - tab.first_block[t]) * kAdamTile;
    const int64_t n = tab.n[t];
    const float gmul = grad_mul != nullptr ? *grad_mul : 1.0f;
    float* __restrict__ P = tab.p[t];
    const GradT* __restrict__ G = static_cast<const GradT*>(tab.g[t]);
    float* __restrict__ M = tab.m[t];
    float* __restrict__ V = tab.v[t];

    if (tab.vec_ok[t] && base + kAdamTile <= n) {
        f32x4 pv[kAdamUnroll], gv[kAdamUnroll], mv[kAdamUnroll], vv[kAdamUnroll];
#pragma unroll
        for (int u = 0; u < kAdamUnroll; ++u) {
            const int64_t e = base + (int64_t(u) * kAdamBlock + threadIdx.x) * 4;
            gv[u] = ld_grad4_nt(G + e);
            wait_vmem();
            mv[u] = ld4_nt(M + e);
            wait_vmem();
            vv[u] = ld4_nt(V + e);
            wait_vmem();
            pv[u] = ld4_nt(P + e);
        }
#pragma unroll
        for (int u = 0; u < kAdamUnroll; ++u) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                float p = pv[u][c], m = mv[u][c], v = vv[u][c];
                adamw_update<kLerpSmall, kUnscale>(p, gv[u][c], m, v, gmul, s);
                pv[u][c] = p;
                mv[u][c] = m;
                vv[u][c] = v;
            }
        }
#pragma unroll
        for (int u = 0; u < kAdamUnroll; ++u) {
            const int64_t e = base + (int64_t(u) * kAdamBlock + threadIdx.x) * 4;
            st4_nt(M + e, mv[u]);
            st4_nt(V + e, vv[u]);
            st4_nt(P + e, pv[u]);
        }
    } else {
        const int64_t end = base + kAdamTile < n ? base + kAdamTile : n;
        for (int64_t e = base + threadIdx.x; e < end; e += kAdamBlock) {
            float p = P[e], m = M[e], v = V[e];
            adamw_update<kLerpSmall, kUnscale>(p, ld_grad1(G + e), m, v, gmul, s);
            P[e] = p;
            M[e] = m;
            V[e] = v;
        }
    }
}

// ---- SGD -------------------------------------------------------------------------
// torch's single-tensor SGD (torch/optim/sgd.py, _single_tensor_sgd) per element, with
// the unscale and clip multiplies in front.  Every `x.add(y, alpha=a)` of torch's CPU
// path is one fused multiply-add, fma(y, a, x); mul_ is one rounded multiply.
enum SgdMode { kSgdPlain = 0, kSgdFirst = 1, kSgdMomentum = 2 };

struct SgdTable {
    float* p[kMaxT];
    const void* g[kMaxT];
    float* buf[kMaxT];
    int64_t n[kMaxT];
    int64_t first_block[kMaxT + 1];
    int32_t vec_ok[kMaxT];
    int32_t count;
};

struct SgdScalars {
    float unscale;
    float weight_decay;
    float momentum;
    float one_minus_dampening;
    float neg_lr;
    int32_t apply_weight_decay;
    int32_t nesterov;
};

template <bool kUnscale, int kMode>
__device__ __forceinline__ void sgd_update(float& p, float g, float& buf, float gmul, const SgdScalars& s) {
    if constexpr (kUnscale) g = g * s.unscale;
    g = g * gmul;
    if (s.apply_weight_decay) g = __builtin_fmaf(p, s.weight_decay, g);  // grad.add(param, alpha=wd)
    if constexpr (kMode == kSgdFirst) {
        buf = g;  // the buffer starts as a clone of the gradient
    } else if constexpr (kMode == kSgdMomentum) {
        buf = buf * s.momentum;
        buf = __builtin_fmaf(g, s.one_minus_dampening, buf);  // buf.mul_(m).add_(grad, alpha=1-d)
    }
    if constexpr (kMode != kSgdPlain) g = s.nesterov ? __builtin_fmaf(buf, s.momentum, g) : buf;
    p = __builtin_fmaf(g, s.neg_lr, p);  // param.add_(grad, alpha=-lr)
}

template <typename GradT, bool kUnscale, int kMode>
__global__ __launch_bounds__(kAdamBlock) void sgd_kernel(SgdTable tab, SgdScalars s,
                                                         const float* __restrict__ grad_mul) {
    const int64_t block = blockIdx.x;
    int t = 0;
    while (t + 1 < tab.count && block >= tab.first_block[t + 1]) ++t;
    const int64_t base = (block - tab.first_block[t]) * kAdamTile;
    const int64_t n = tab.n[t];
    const float gmul = grad_mul != nullptr ? *grad_mul : 1.0f;
    float* __restrict__ P = tab.p[t];
    const GradT* __restrict__ G = static_cast<const GradT*>(tab.g[t]);
    float* __restrict__ B = tab.buf[t];
    if (tab.vec_ok[t] && base + kAdamTile <= n) {
        f32x4 pv[kAdamUnroll], gv[kAdamUnroll], bv[kAdamUnroll];
#pragma unroll
        for (int u = 0; u < kAdamUnroll; ++u) {
            const int64_t e = base + (int64_t(u) * kAdamBlock + threadIdx.x) * 4;
            gv[u] = ld_grad4_nt(G + e);
            if constexpr (kMode == kSgdMomentum) {
                wait_vmem();
                bv[u] = ld4_nt(B + e);
            }
            wait_vmem();
            pv[u] = ld4_nt(P + e);
        }
#pragma unroll
        for (int u = 0; u < kAdamUnroll; ++u) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                float p = pv[u][c], b = kMode == kSgdMomentum ? bv[u][c] : 0.0f;
                sgd_update<kUnscale, kMode>(p, gv[u][c], b, gmul, s);
                pv[u][c] = p;
                bv[u][c] = b;
            }
        }
#pragma unroll
        for (int u = 0; u < kAdamUnroll; ++u) {
            const int64_t e = base + (int64_t(u) * kAdamBlock + threadIdx.x) * 4;
            if constexpr (kMode != kSgdPlain) st4_nt(B + e, bv[u]);
            st4_nt(P + e, pv[u]);
        }
    } else {
        const int64_t end = base + kAdamTile < n ? base + kAdamTile : n;
        for (int64_t e = base + threadIdx.x; e < end; e += kAdamBlock) {
            float p = P[e], b = kMode == kSgdMomentum ? B[e] : 0.0f;
            sgd_update<kUnscale, kMode>(p, ld_grad1(G + e), b, gmul, s);
            P[e] = p;
            if constexpr (kMode != kSgdPlain) B[e] = b;
        }
    }
}

// ---- squared norm ------------------------------------------------------------------
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

// Workgroup c sums chunk c of the concatenated tensors (8 tiles of one tensor: 32768
// fp32 or 65536 bf16 elements) into partials[c].  Inside a thread the squares are added in element order;
// threads and waves are combined by the fixed trees of block_sum, so the partials,
// and the sum of them, depend only on the data and the numels.
template <typename GradT, bool kUnscale>
__global__ __launch_bounds__(kNormBlock) void sqnorm_kernel(NormTable tab, float unscale,
                                                            double* __restrict__ partials) {
    constexpr int64_t kTile = norm_tile<GradT>();
    constexpr int64_t kChunk = norm_chunk<GradT>();
    const int64_t chunk = blockIdx.x;
    int t = 0;
    while (t + 1 < tab.count && chunk >= tab.first_chunk[t + 1]) ++t;
    const int64_t start = (chunk - tab.first_chunk[t]) * kChunk;
    const int64_t n = tab.n[t];
    const GradT* __restrict__ G = static_cast<const GradT*>(tab.g[t]);
    double acc = 0.0;
    for (int k = 0; k < kNormTilesPerChunk; ++k) {
        const int64_t base = start + int64_t(k) * kTile;
        if (base >= n) break;
        if (tab.vec_ok[t] && base + kTile <= n) {
            f32x4 x, y;
            if constexpr (sizeof(GradT) == 4) {
                x = ld_grad4_nt(G + base + int64_t(threadIdx.x) * 4);
            } else {
                ld_bf16x8_nt(G + base + int64_t(threadIdx.x) * 8, x, y);
            }
            if constexpr (kUnscale) x = x * unscale;
            acc += sq(x.x);
            acc += sq(x.y);
            acc += sq(x.z);
            acc += sq(x.w);
            if constexpr (sizeof(GradT) == 2) {
                if constexpr (kUnscale) y = y * unscale;
                acc += sq(y.x);
                acc += sq(y.y);
                acc += sq(y.z);
                acc += sq(y.w);
            }
        } else {
            const int64_t end = base + kTile < n ? base + kTile : n;
            for (int64_t e = base + threadIdx.x; e < end; e += kNormBlock) {
                float x = ld_grad1(G + e);
                if constexpr (kUnscale) x = x * unscale;
                acc += sq(x);
            }
        }
    }
    const double block_total = block_sum<kNormBlock>(acc);
    if (threadIdx.x == 0) partials[chunk] = block_total * tab.w[t];
}

// ---- FSDP gradient local share fused with the norm partials -----------------------
// Writes the rank's fp32 gradient shard exactly as the local-share kernel does (sum
// over ranks, in rank order, of fp32(x_q) / divisor; +0.0 over the padding tail) and,
// in the same pass, the squared norm of every 256-element tile of it.  A second,
// small kernel adds each 128 consecutive tile sums into one partial per 32768-element
// chunk of the segments [0, valid) and [valid, shard), the layout the norm pass uses,
// so the optimizer can take them in its place.  Every sum has a fixed order: per lane
// the 4 squares in element order, per tile a butterfly over the 64 lanes, per chunk
// lane l's pair (tile l, tile l + 64) then a butterfly.
struct ShareRanks {
    const uint8_t* g[HBT_MAX_LOCAL_RANKS];
};

constexpr int kShareBlock = 64;
constexpr int64_t kShareTile = int64_t(kShareBlock) * 4;  // 256 elements, one wave
constexpr int64_t kTilesPerNormChunk = norm_chunk<float>() / kShareTile;  // 128

// Loads of one rank's gradient widened to fp32: SB-byte elements, a 2-byte element
// being bf16, or IEEE fp16 when H is set.
template <int SB, bool H>
__device__ __forceinline__ float share_load1(const uint8_t* p) {
    if constexpr (SB == 4) return *reinterpret_cast<const float*>(p);
    return b16_to_f32<H>(*reinterpret_cast<const uint16_t*>(p));
}

// Division by a power of two is exact scaling, so x / d == x * (1 / d) bitwise for
// every x (both are the correctly rounded x * 2^-k); other divisors divide.
template <bool kRecip>
__device__ __forceinline__ f32x4 share_div(f32x4 x, float divisor, float recip) {
    if constexpr (kRecip) return x * recip;
    return x / divisor;
}
template <bool kRecip>
__device__ __forceinline__ float share_div1(float x, float divisor, float recip) {
    if constexpr (kRecip) return x * recip;
    return x / divisor;
}
template <int SB, bool H>
__device__ __forceinline__ f32x4 share_load4(const uint8_t* p) {
    if constexpr (SB == 4) {
        return ld4_nt(reinterpret_cast<const float*>(p));
    } else if constexpr (H) {
        const u32x2 w = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
        return f32x4{f16_to_f32(w.x & 0xFFFFu), f16_to_f32(w.x >> 16), f16_to_f32(w.y & 0xFFFFu),
                     f16_to_f32(w.y >> 16)};
    } else {
        return ld_grad4_nt(reinterpret_cast<const uint16_t*>(p));
    }
}

// The reduce dtype's steps of the reference's AVG reduce-scatter (RD: the dtype code).
// The gradient is cast to RD unless it already has that dtype (Tensor.to), each
// division and each addition is rounded to RD (torch computes them in fp32 and rounds
// once), and the result widens exactly to the fp32 master.  For RD = F32 every step is
// the identity, so the fp32 instantiations are the plain fp32 local share.
template <int RD>
__device__ __forceinline__ f32x4 round4(f32x4 v) {
    if constexpr (RD == HBT_DTYPE_F32) return v;
    return f32x4{round_to<RD>(v.x), round_to<RD>(v.y), round_to<RD>(v.z), round_to<RD>(v.w)};
}
template <int SB, bool H, int RD>
__device__ __forceinline__ f32x4 share_cast4(f32x4 x) {
    if constexpr (dtype_of<SB, H>() == RD) return x;
    return round4<RD>(x);
}
template <int SB, bool H, int RD>
__device__ __forceinline__ float share_cast1(float x) {
    if constexpr (dtype_of<SB, H>() == RD) return x;
    return round_to<RD>(x);
}

// One wave per 256-element tile: measured on MI355X (8 bf16 ranks -> fp32) this
// short-lived shape streams at 6.4 TB/s, against 5.6 TB/s for the norm kernel's
// 1024-thread, 8-tile workgroups.  kG > 0 fixes the group size so that every rank's
// load is issued before the first is used; kG == 0 reads group_size at run time.
template <int SB, int kG, bool kRecip, bool H, int RD>
__global__ __launch_bounds__(kShareBlock) void local_share_tiles_kernel(
    ShareRanks ranks, int32_t group_size, int64_t offset, int64_t shard_numel, int64_t valid_numel,
    float divisor, float recip, int32_t vec_ok, float* __restrict__ out, double* __restrict__ tile_sums) {
    const int64_t base = int64_t(blockIdx.x) * kShareTile;
    double acc = 0.0;
    if (vec_ok && base + kShareTile <= valid_numel) {
        const int64_t e = base + int64_t(threadIdx.x) * 4;
        f32x4 sum;
        if constexpr (kG > 0) {
            f32x4 x[kG];
#pragma unroll
            for (int q = 0; q < kG; ++q) x[q] = share_load4<SB, H>(ranks.g[q] + (offset + e) * SB);
            sum = round4<RD>(share_div<kRecip>(share_cast4<SB, H, RD>(x[0]), divisor, recip));
#pragma unroll
            for (int q = 1; q < kG; ++q) {
                sum = round4<RD>(sum + round4<RD>(share_div<kRecip>(share_cast4<SB, H, RD>(x[q]), divisor, recip)));
            }
        } else {
            sum = round4<RD>(share_div<kRecip>(
                share_cast4<SB, H, RD>(share_load4<SB, H>(ranks.g[0] + (offset + e) * SB)), divisor, recip));
            for (int32_t q = 1; q < group_size; ++q) {
                const f32x4 x = share_cast4<SB, H, RD>(share_load4<SB, H>(ranks.g[q] + (offset + e) * SB));
                sum = round4<RD>(sum + round4<RD>(share_div<kRecip>(x, divisor, recip)));
            }
        }
        st4_nt(out + e, sum);
        acc += sq(sum.x);
        acc += sq(sum.y);
        acc += sq(sum.z);
        acc += sq(sum.w);
    } else if (vec_ok && base >= valid_numel && base + kShareTile <= shard_numel) {
        st4_nt(out + base + int64_t(threadIdx.x) * 4, f32x4{0.0f, 0.0f, 0.0f, 0.0f});
    } else {
        const int64_t end = base + kShareTile < shard_numel ? base + kShareTile : shard_numel;
        for (int64_t e = base + threadIdx.x; e < end; e += kShareBlock) {
            float v = 0.0f;
            if (e < valid_numel) {
                v = round_to<RD>(share_div1<kRecip>(
                    share_cast1<SB, H, RD>(share_load1<SB, H>(ranks.g[0] + (offset + e) * SB)), divisor, recip));
                for (int32_t q = 1; q < group_size; ++q) {
                    const float x = share_cast1<SB, H, RD>(share_load1<SB, H>(ranks.g[q] + (offset + e) * SB));
                    v = round_to<RD>(v + round_to<RD>(share_div1<kRecip>(x, divisor, recip)));
                }
            }
            out[e] = v;
            acc += sq(v);
        }
    }
    acc = wave_sum(acc);
    if (threadIdx.x == 0) tile_sums[blockIdx.x] = acc;
}

// Reduce dtype float64: each rank's element widens exactly to double (SB = 8 reads a
// float64 no_sync accumulator), the divide and the rank-order sum run in double, both
// correctly rounded as torch's float64 div and add are, and the sum rounds once, to
// nearest even, to the fp32 master (Tensor.to).  Lane l owns elements 4l .. 4l + 3 of
// its tile, so the tile sums add the squares in the fp32 kernel's order.
template <int SB, bool H>
__global__ __launch_bounds__(kShareBlock) void local_share_f64_tiles_kernel(
    ShareRanks ranks, int32_t group_size, int64_t offset, int64_t shard_numel, int64_t valid_numel,
    double divisor, float* __restrict__ out, double* __restrict__ tile_sums) {
    const int64_t first = int64_t(blockIdx.x) * kShareTile + int64_t(threadIdx.x) * 4;
    double acc = 0.0;
    for (int j = 0; j < 4; ++j) {
        const int64_t e = first + j;
        if (e >= shard_numel) break;
        float v = 0.0f;
        if (e < valid_numel) {
            double s = widen_f64<SB, H>(ranks.g[0], offset + e) / divisor;
            for (int32_t q = 1; q < group_size; ++q) s = s + widen_f64<SB, H>(ranks.g[q], offset + e) / divisor;
            v = static_cast<float>(s);
        }
        out[e] = v;
        acc += sq(v);
    }
    acc = wave_sum(acc);
    if (threadIdx.x == 0) tile_sums[blockIdx.x] = acc;
}

// Chunk c < valid_chunks: the sum of tile sums 128c .. 128c + 127 (those below
// valid_tiles); padding chunks: 0, the square sum of zeros.
__global__ __launch_bounds__(kShareBlock) void tile_sums_to_partials_kernel(
    const double* __restrict__ tile_sums, int64_t valid_tiles, int64_t valid_chunks,
    double* __restrict__ partials) {
    const int64_t chunk = blockIdx.x;
    double acc = 0.0;
    if (chunk < valid_chunks) {
        const int64_t first = chunk * kTilesPerNormChunk;
        const int64_t a = first + threadIdx.x;
        const int64_t b = a + kShareBlock;
        if (a < valid_tiles) acc = tile_sums[a];
        if (b < valid_tiles) acc += tile_sums[b];
    }
    acc = wave_sum(acc);
    if (threadIdx.x == 0) partials[chunk] = acc;
}

constexpr int kFinalBlock = 1024;

__global__ __launch_bounds__(kFinalBlock) void norm_finalize_kernel(
    const double* __restrict__ partials, int64_t count, double max_norm, double* __restrict__ sum_out,
    double* __restrict__ norm_out, float* __restrict__ grad_mul_out, int32_t* __restrict__ nonfinite_out) {
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
    if (grad_mul_out != nullptr) {
        float mul = 1.0f;
        if (max_norm > 0.0) {
            const double coef = max_norm / (norm + 1e-6);
            if (coef < 1.0) mul = static_cast<float>(coef);
        }
        grad_mul_out[0] = mul;
    }
    if (nonfinite_out != nullptr) nonfinite_out[0] = isfinite(total) ? 0 : 1;
}

// ---- in-place scaling ---------------------------------------------------------------
// Half-wave (32-thread) workgroups, two 16-byte vectors per lane: 256 fp32 or 512 bf16
// elements per workgroup.  Measured on MI355X (in-place, 1e9 fp32): 6.8 TB/s, against
// 6.0 TB/s for 64 threads with one vector and 5.5 TB/s with two.
constexpr int kScaleBlock = 32;
template <typename T>
constexpr int64_t scale_tile() { return int64_t(kScaleBlock) * 2 * (16 / sizeof(T)); }

struct ScaleTable {
    void* x[kMaxT];
    int64_t n[kMaxT];
    int64_t first_block[kMaxT + 1];
    int32_t vec_ok[kMaxT];
    int32_t count;
};

template <typename T>
__device__ __forceinline__ float to_f32(T x);
template <>
__device__ __forceinline__ float to_f32<float>(float x) { return x; }
template <>
__device__ __forceinline__ float to_f32<uint16_t>(uint16_t x) { return bf16_to_f32(x); }
template <typename T>
__device__ __forceinline__ T from_f32(float x);
template <>
__device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <>
__device__ __forceinline__ uint16_t from_f32<uint16_t>(float x) {
    return static_cast<uint16_t>(f32_to_bf16(x));
}

// Two separate multiplies, each rounded to T, as two in-place mul_ calls would do.
template <typename T>
__device__ __forceinline__ T scale_one(T x, float unscale, float mul) {
    const T y = from_f32<T>(to_f32<T>(x) * unscale);
    return from_f32<T>(to_f32<T>(y) * mul);
}

template <typename T>
__global__ __launch_bounds__(kScaleBlock) void scale_kernel(ScaleTable tab, float unscale,
                                                            const float* __restrict__ grad_mul) {
    const int64_t block = blockIdx.x;
    int t = 0;
    while (t + 1 < tab.count && block >= tab.first_block[t + 1]) ++t;
    constexpr int64_t kTile = scale_tile<T>();
    const int64_t base = (block - tab.first_block[t]) * kTile;
    const int64_t n = tab.n[t];
    const float mul = grad_mul != nullptr ? *grad_mul : 1.0f;
    T* __restrict__ x = static_cast<T*>(tab.x[t]);
    typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
    if (tab.vec_ok[t] && base + kTile <= n) {
        if constexpr (sizeof(T) == 4) {
            f32x4 v[2];
            float* p[2];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                p[u] = reinterpret_cast<float*>(x) + base + (int64_t(u) * kScaleBlock + threadIdx.x) * 4;
                v[u] = ld4_nt(p[u]);
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
#pragma unroll
                for (int c = 0; c < 4; ++c) v[u][c] = scale_one<float>(v[u][c], unscale, mul);
                st4_nt(p[u], v[u]);
            }
        } else {
            u32x4v w[2];
            uint16_t* p[2];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                p[u] = reinterpret_cast<uint16_t*>(x) + base + (int64_t(u) * kScaleBlock + threadIdx.x) * 8;
                w[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4v*>(p[u]));
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const uint32_t lo = scale_one<uint16_t>(static_cast<uint16_t>(w[u][c] & 0xFFFFu), unscale, mul);
                    const uint32_t hi = scale_one<uint16_t>(static_cast<uint16_t>(w[u][c] >> 16), unscale, mul);
                    w[u][c] = lo | (hi << 16);
                }
                __builtin_nontemporal_store(w[u], reinterpret_cast<u32x4v*>(p[u]));
            }
        }
        return;
    }
    const int64_t end = base + kTile < n ? base + kTile : n;
    for (int64_t i = base + threadIdx.x; i < end; i += kScaleBlock) x[i] = scale_one<T>(x[i], unscale, mul);
}

// ---- no_sync gradient accumulation ----------------------------------------------------
// acc = R(acc + R(grad)), R rounding to the accumulator's dtype (the reduce dtype): the
// gradient's cast to that dtype (Tensor.to) and one addition computed in fp32 and
// rounded once (add_).  kAssign writes R(grad) instead: the first micro-batch's clone.
// The scale kernel's shape: half-wave workgroups, two 4-element vectors per lane,
// 256 accumulator elements per workgroup.
constexpr int64_t kAccumTile = int64_t(kScaleBlock) * 2 * 4;

struct AccumTable {
    void* acc[kMaxT];
    const void* grad[kMaxT];
    int64_t n[kMaxT];
    int64_t first_block[kMaxT + 1];
    int32_t vec_ok[kMaxT];
    int32_t count;
};

// Four elements of B bytes each (fp32, or bf16 / fp16 when H), widened exactly.
template <int B, bool H>
__device__ __forceinline__ f32x4 load4_as_f32(const unsigned char* p) {
    if constexpr (B == 4) {
        return ld4_nt(reinterpret_cast<const float*>(p));
    } else {
        const u32x2 w = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
        return f32x4{b16_to_f32<H>(w.x & 0xFFFFu), b16_to_f32<H>(w.x >> 16), b16_to_f32<H>(w.y & 0xFFFFu),
                     b16_to_f32<H>(w.y >> 16)};
    }
}
// Four values already representable in the B-byte dtype, stored in it.
template <int B, bool H>
__device__ __forceinline__ void store4_from_f32(unsigned char* p, f32x4 v) {
    if constexpr (B == 4) {
        st4_nt(reinterpret_cast<float*>(p), v);
    } else {
        const u32x2 w{f32_to_b16<H>(v.x) | (f32_to_b16<H>(v.y) << 16), f32_to_b16<H>(v.z) | (f32_to_b16<H>(v.w) << 16)};
        __builtin_nontemporal_store(w, reinterpret_cast<u32x2*>(p));
    }
}
template <int B, bool H>
__device__ __forceinline__ float load1_as_f32(const unsigned char* p, int64_t i) {
    if constexpr (B == 4) return reinterpret_cast<const float*>(p)[i];
    return b16_to_f32<H>(reinterpret_cast<const uint16_t*>(p)[i]);
}
template <int B, bool H>
__device__ __forceinline__ void store1_from_f32(unsigned char* p, int64_t i, float v) {
    if constexpr (B == 4) {
        reinterpret_cast<float*>(p)[i] = v;
    } else {
        reinterpret_cast<uint16_t*>(p)[i] = static_cast<uint16_t>(f32_to_b16<H>(v));
    }
}

// SB/SH: the gradient's element size and fp16 flag; AB/AH: the accumulator's.
template <int SB, bool SH, int AB, bool AH, bool kAssign>
__global__ __launch_bounds__(kScaleBlock) void accumulate_kernel(AccumTable tab) {
    constexpr int RD = dtype_of<AB, AH>();
    const int64_t block = blockIdx.x;
    int t = 0;
    while (t + 1 < tab.count && block >= tab.first_block[t + 1]) ++t;
    const int64_t base = (block - tab.first_block[t]) * kAccumTile;
    const int64_t n = tab.n[t];
    unsigned char* __restrict__ acc = static_cast<unsigned char*>(tab.acc[t]);
    const unsigned char* __restrict__ grad = static_cast<const unsigned char*>(tab.grad[t]);
    if (tab.vec_ok[t] && base + kAccumTile <= n) {
        f32x4 a[2], g[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int64_t i = base + (int64_t(u) * kScaleBlock + threadIdx.x) * 4;
            g[u] = share_cast4<SB, SH, RD>(load4_as_f32<SB, SH>(grad + i * SB));
        }
        if constexpr (!kAssign) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int64_t i = base + (int64_t(u) * kScaleBlock + threadIdx.x) * 4;
                a[u] = load4_as_f32<AB, AH>(acc + i * AB);
            }
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int64_t i = base + (int64_t(u) * kScaleBlock + threadIdx.x) * 4;
            if constexpr (kAssign) {
                store4_from_f32<AB, AH>(acc + i * AB, g[u]);
            } else {
                store4_from_f32<AB, AH>(acc + i * AB, round4<RD>(a[u] + g[u]));
            }
        }
        return;
    }
    const int64_t end = base + kAccumTile < n ? base + kAccumTile : n;
    for (int64_t i = base + threadIdx.x; i < end; i += kScaleBlock) {
        const float g = share_cast1<SB, SH, RD>(load1_as_f32<SB, SH>(grad, i));
        if constexpr (kAssign) {
            store1_from_f32<AB, AH>(acc, i, g);
        } else {
            store1_from_f32<AB, AH>(acc, i, round_to<RD>(load1_as_f32<AB, AH>(acc, i) + g));
        }
    }
}

inline bool aligned(const void* ptr, uintptr_t bytes) {
    return (reinterpret_cast<uintptr_t>(ptr) % bytes) == 0;
}


// ---- norm launch helpers (shared by the workspace and the no-allocation entry points) --
// Validates a gradient table and fills the norm kernel's table; `chunks` is the number
// of partials the launch writes.
int32_t build_norm_table(const char* who, const void* const* grads, const int64_t* numels,
                         const double* weights, int32_t count, int32_t grad_dtype, NormTable& tab,
                         int64_t& chunks) {
    if (count < 0 || count > kMaxT) {
        set_error("%s: count must lie in [0, %d], got %d", who, kMaxT, count);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if (grad_dtype != HBT_DTYPE_F32 && grad_dtype != HBT_DTYPE_BF16) {
        set_error("%s: gradient dtype %d is not F32 or BF16", who, grad_dtype);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if (count > 0 && (grads == nullptr || numels == nullptr || weights == nullptr)) {
        set_error("%s: null pointer argument", who);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    tab = NormTable{};
    tab.count = count;
    const int64_t kChunk = grad_dtype == HBT_DTYPE_F32 ? norm_chunk<float>() : norm_chunk<uint16_t>();
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

// One sqnorm_kernel launch writing partials[0, chunks).
int32_t launch_sqnorm(const char* who, const NormTable& tab, int64_t chunks, int32_t grad_dtype, float unscale,
                      double* partials, hipStream_t st) {
    if (chunks == 0) return HBT_OK;
    if (chunks > 0x7FFFFFFFLL) {
        set_error("%s: %lld chunks exceed the grid limit", who, static_cast<long long>(chunks));
        return HBT_ERR_UNSUPPORTED;
    }
    const dim3 grid(static_cast<unsigned>(chunks));
    const bool scaled = unscale != 1.0f;
    if (grad_dtype == HBT_DTYPE_F32) {
        if (scaled) {
            sqnorm_kernel<float, true><<<grid, kNormBlock, 0, st>>>(tab, unscale, partials);
        } else {
            sqnorm_kernel<float, false><<<grid, kNormBlock, 0, st>>>(tab, unscale, partials);
        }
    } else {
        if (scaled) {
            sqnorm_kernel<uint16_t, true><<<grid, kNormBlock, 0, st>>>(tab, unscale, partials);
        } else {
            sqnorm_kernel<uint16_t, false><<<grid, kNormBlock, 0, st>>>(tab, unscale, partials);
        }
    }
    return check_launch(who);
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

}  // namespace
}  // namespace hbt

using namespace hbt;

// Accumulator float64: the gradient widens exactly (Tensor.to) and each add runs in
// double, as add_ on float64 tensors does; kAssign writes the widened gradient.
template <int SB, bool SH, bool kAssign>
__global__ __launch_bounds__(kScaleBlock) void accumulate_f64_kernel(AccumTable tab) {
    const int64_t block = blockIdx.x;
    int t = 0;
    while (t + 1 < tab.count && block >= tab.first_block[t + 1]) ++t;
    const int64_t base = (block - tab.first_block[t]) * kAccumTile;
    const int64_t n = tab.n[t];
    double* __restrict__ acc = static_cast<double*>(tab.acc[t]);
    const unsigned char* __restrict__ grad = static_cast<const unsigned char*>(tab.grad[t]);
    const int64_t end = base + kAccumTile < n ? base + kAccumTile : n;
    for (int64_t i = base + threadIdx.x; i < end; i += kScaleBlock) {
        const double g = widen_f64<SB, SH>(grad, i);
        acc[i] = kAssign ? g : acc[i] + g;
    }
}

extern "C" {

int32_t hbt_adamw_step(float* const* params, const void* const* grads, float* const* exp_avgs,
                       float* const* exp_avg_sqs, const int64_t* numels, int32_t count,
                       int32_t grad_dtype, float unscale, const float* grad_mul, float decay,
                       float lerp_weight, float beta2, float one_minus_beta2,
                       float bias_correction2_sqrt, float eps, float neg_step_size, void* stream) {
    clear_error();
    if (count < 0 || count > kMaxT) {
        set_error("hbt_adamw_step: count must lie in [0, %d], got %d", kMaxT, count);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if (grad_dtype != HBT_DTYPE_F32 && grad_dtype != HBT_DTYPE_BF16) {
        set_error("hbt_adamw_step: gradient dtype %d is not F32 or BF16", grad_dtype);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if (count > 0 && (params == nullptr || grads == nullptr || exp_avgs == nullptr ||
                      exp_avg_sqs == nullptr || numels == nullptr)) {
        set_error("hbt_adamw_step: null table pointer");
        return HBT_ERR_INVALID_ARGUMENT;
    }
    AdamTable tab{};
    tab.count = count;
    const uintptr_t grad_align = grad_dtype == HBT_DTYPE_F32 ? 16 : 8;
    int64_t blocks = 0;
    for (int i = 0; i < count; ++i) {
        if (numels[i] < 0) {
            set_error("hbt_adamw_step: tensor %d has negative numel %lld", i,
                      static_cast<long long>(numels[i]));
            return HBT_ERR_INVALID_ARGUMENT;
        }
        if (numels[i] > 0 && (params[i] == nullptr || grads[i] == nullptr || exp_avgs[i] == nullptr ||
                              exp_avg_sqs[i] == nullptr)) {
            set_error("hbt_adamw_step: tensor %d has a null data pointer", i);
            return HBT_ERR_INVALID_ARGUMENT;
        }
        tab.p[i] = params[i];
        tab.g[i] = grads[i];
        tab.m[i] = exp_avgs[i];
        tab.v[i] = exp_avg_sqs[i];
        tab.n[i] = numels[i];
        tab.vec_ok[i] = aligned(params[i], 16) && aligned(grads[i], grad_align) &&
                        aligned(exp_avgs[i], 16) && aligned(exp_avg_sqs[i], 16);
        tab.first_block[i] = blocks;
        blocks += (numels[i] + kAdamTile - 1) / kAdamTile;
    }
    tab.first_block[count] = blocks;
    for (int i = count + 1; i <= kMaxT; ++i) tab.first_block[i] = blocks;
    if (blocks == 0) return HBT_OK;
    if (blocks > 0x7FFFFFFFLL) {
        set_error("hbt_adamw_step: %lld tiles exceed the grid limit", static_cast<long long>(blocks));
        return HBT_ERR_UNSUPPORTED;
    }
    AdamScalars s{};
    s.unscale = unscale;
    s.decay = decay;
    s.lerp_w = lerp_weight;
    s.lerp_w_minus_1 = lerp_weight - 1.0f;
    s.beta2 = beta2;
    s.one_minus_beta2 = one_minus_beta2;
    s.bc2_sqrt = bias_correction2_sqrt;
    s.eps = eps;
    s.neg_step = neg_step_size;
    const bool lerp_small = std::fabs(lerp_weight) < 0.5f;
    const bool scaled = unscale != 1.0f;
    const dim3 grid(static_cast<unsigned>(blocks));
    hipStream_t st = as_stream(stream);
#define HBT_ADAMW_LAUNCH(GT, SMALL, SCALED) \
    adamw_kernel<GT, SMALL, SCALED><<<grid, kAdamBlock, 0, st>>>(tab, s, grad_mul)
    if (grad_dtype == HBT_DTYPE_F32) {
        if (lerp_small) {
            if (scaled) HBT_ADAMW_LAUNCH(float, true, true); else HBT_ADAMW_LAUNCH(float, true, false);
        } else {
            if (scaled) HBT_ADAMW_LAUNCH(float, false, true); else HBT_ADAMW_LAUNCH(float, false, false);
        }
    } else {
        if (lerp_small) {
            if (scaled) HBT_ADAMW_LAUNCH(uint16_t, true, true); else HBT_ADAMW_LAUNCH(uint16_t, true, false);
        } else {
            if (scaled) HBT_ADAMW_LAUNCH(uint16_t, false, true); else HBT_ADAMW_LAUNCH(uint16_t, false, false);
        }
    }
#undef HBT_ADAMW_LAUNCH
    return check_launch("hbt_adamw_step");
}

int64_t hbt_norm_partials_count(const int64_t* numels, int32_t count, int32_t grad_dtype) {
    if (count < 0 || count > kMaxT || (count > 0 && numels == nullptr)) return -1;
    if (grad_dtype != HBT_DTYPE_F32 && grad_dtype != HBT_DTYPE_BF16) return -1;
    const int64_t chunk = grad_dtype == HBT_DTYPE_F32 ? norm_chunk<float>() : norm_chunk<uint16_t>();
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
    NormTable tab{};
    int64_t chunks = 0;
    const int32_t status = build_norm_table("hbt_grad_sqnorm_partials", grads, numels, weights, count,
                                            grad_dtype, tab, chunks);
    if (status != HBT_OK) return status;
    return launch_sqnorm("hbt_grad_sqnorm_partials", tab, chunks, grad_dtype, unscale, partials,
                         as_stream(stream));
}

int32_t hbt_grad_norm_finalize(const double* partials, int64_t count, double max_norm,
                               double* sum_out, double* norm_out, float* grad_mul_out,
                               int32_t* nonfinite_out, void* stream) {
    clear_error();
    if (count < 0 || (count > 0 && partials == nullptr)) {
        set_error("hbt_grad_norm_finalize: bad partials/count");
        return HBT_ERR_INVALID_ARGUMENT;
    }
    norm_finalize_kernel<<<1, kFinalBlock, 0, as_stream(stream)>>>(partials, count, max_norm, sum_out,
                                                                   norm_out, grad_mul_out, nonfinite_out);
    return check_launch("hbt_grad_norm_finalize");
}

int32_t hbt_grad_norm_noalloc(const void* const* grads, const int64_t* numels, const double* weights,
                              int32_t count, int32_t grad_dtype, float unscale, double max_norm,
                              double* sum_out, double* norm_out, float* grad_mul_out,
                              int32_t* nonfinite_out, void* stream) {
    clear_error();
    NormTable tab{};
    int64_t chunks = 0;
    int32_t status = build_norm_table("hbt_grad_norm_noalloc", grads, numels, weights, count, grad_dtype,
                                      tab, chunks);
    if (status != HBT_OK) return status;
    if (chunks > HBT_NOALLOC_MAX_PARTIALS) {
        set_error("hbt_grad_norm_noalloc: the gradients need %lld norm partials, more than the %d the "
                  "static scratch holds (at most %lld fp32 or %lld bf16 elements per call)",
                  static_cast<long long>(chunks), HBT_NOALLOC_MAX_PARTIALS,
                  static_cast<long long>(HBT_NOALLOC_MAX_PARTIALS * norm_chunk<float>()),
                  static_cast<long long>(HBT_NOALLOC_MAX_PARTIALS * norm_chunk<uint16_t>()));
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
                                                   grad_mul_out, nonfinite_out);
    return check_launch("hbt_grad_norm_noalloc");
}

int32_t hbt_scale_inplace(void* const* tensors, const int64_t* numels, int32_t count,
                          int32_t dtype, float unscale, const float* grad_mul, void* stream) {
    clear_error();
    if (count < 0 || count > kMaxT || (count > 0 && (tensors == nullptr || numels == nullptr))) {
        set_error("hbt_scale_inplace: bad table (count=%d)", count);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if (dtype != HBT_DTYPE_F32 && dtype != HBT_DTYPE_BF16) {
        set_error("hbt_scale_inplace: dtype %d is not F32 or BF16", dtype);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    ScaleTable tab{};
    tab.count = count;
    const int64_t tile = dtype == HBT_DTYPE_F32 ? scale_tile<float>() : scale_tile<uint16_t>();
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
    if (blocks == 0) return HBT_OK;
    if (blocks > 0x7FFFFFFFLL) {
        set_error("hbt_scale_inplace: %lld tiles exceed the grid limit", static_cast<long long>(blocks));
        return HBT_ERR_UNSUPPORTED;
    }
    if (dtype == HBT_DTYPE_F32) {
        scale_kernel<float><<<dim3(static_cast<unsigned>(blocks)), kScaleBlock, 0, as_stream(stream)>>>(
            tab, unscale, grad_mul);
    } else {
        scale_kernel<uint16_t><<<dim3(static_cast<unsigned>(blocks)), kScaleBlock, 0, as_stream(stream)>>>(
            tab, unscale, grad_mul);
    }
    return check_launch("hbt_scale_inplace");
}

int32_t hbt_grad_accumulate(void* const* accumulators, const void* const* grads, const int64_t* numels,
                            int32_t count, int32_t acc_dtype, int32_t grad_dtype, int32_t flags, void* stream) {
    clear_error();
    if (count < 0 || count > kMaxT ||
        (count > 0 && (accumulators == nullptr || grads == nullptr || numels == nullptr))) {
        set_error("hbt_grad_accumulate: bad table (count=%d)", count);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    const auto float_code = [](int32_t d) {
        return d == HBT_DTYPE_F32 || d == HBT_DTYPE_BF16 || d == HBT_DTYPE_F16;
    };
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
    if (blocks == 0) return HBT_OK;
    if (blocks > 0x7FFFFFFFLL) {
        set_error("hbt_grad_accumulate: %lld tiles exceed the grid limit", static_cast<long long>(blocks));
        return HBT_ERR_UNSUPPORTED;
    }
    const dim3 grid(static_cast<unsigned>(blocks));
    hipStream_t st = as_stream(stream);
    const bool assign = (flags & HBT_ACCUMULATE_ASSIGN) != 0;
#define HBT_ACC(SB, SH, AB, AH)                                                                    \
    do {                                                                                           \
        if (assign) accumulate_kernel<SB, SH, AB, AH, true><<<grid, kScaleBlock, 0, st>>>(tab);    \
        else accumulate_kernel<SB, SH, AB, AH, false><<<grid, kScaleBlock, 0, st>>>(tab);          \
    } while (0)
#define HBT_ACC_A(SB, SH)                                                          \
    do {                                                                           \
        if (acc_dtype == HBT_DTYPE_F32) HBT_ACC(SB, SH, 4, false);                  \
        else if (acc_dtype == HBT_DTYPE_BF16) HBT_ACC(SB, SH, 2, false);            \
        else HBT_ACC(SB, SH, 2, true);                                             \
    } while (0)
#define HBT_ACC64(SB, SH)                                                                    \
    do {                                                                                     \
        if (assign) accumulate_f64_kernel<SB, SH, true><<<grid, kScaleBlock, 0, st>>>(tab);   \
        else accumulate_f64_kernel<SB, SH, false><<<grid, kScaleBlock, 0, st>>>(tab);         \
    } while (0)
    if (f64) {
        if (grad_dtype == HBT_DTYPE_F64) HBT_ACC64(8, false);
        else if (grad_dtype == HBT_DTYPE_F32) HBT_ACC64(4, false);
        else if (grad_dtype == HBT_DTYPE_BF16) HBT_ACC64(2, false);
        else HBT_ACC64(2, true);
    } else if (grad_dtype == HBT_DTYPE_F32) {
        HBT_ACC_A(4, false);
    } else if (grad_dtype == HBT_DTYPE_BF16) {
        HBT_ACC_A(2, false);
    } else {
        HBT_ACC_A(2, true);
    }
#undef HBT_ACC_A
#undef HBT_ACC64
#undef HBT_ACC
    return check_launch("hbt_grad_accumulate");
}


int32_t hbt_grad_local_share_sqnorm(const void* const* rank_grads, int32_t group_size, int32_t rank,
                                    int64_t shard_numel, int64_t valid_numel, int32_t in_dtype,
                                    int32_t reduce_dtype, float divisor, float* out, double* partials,
                                    double* tile_scratch, void* stream) {
    clear_error();
    if (rank_grads == nullptr || out == nullptr || partials == nullptr || tile_scratch == nullptr ||
        group_size < 1 || group_size > HBT_MAX_LOCAL_RANKS || rank < 0 || rank >= group_size ||
        shard_numel < 0 || valid_numel < 0 || valid_numel > shard_numel) {
        set_error("hbt_grad_local_share_sqnorm: bad arguments (group_size=%d rank=%d shard=%lld valid=%lld)",
                  group_size, rank, static_cast<long long>(shard_numel), static_cast<long long>(valid_numel));
        return HBT_ERR_INVALID_ARGUMENT;
    }
    const bool f64 = reduce_dtype == HBT_DTYPE_F64;
    if (in_dtype != HBT_DTYPE_F32 && in_dtype != HBT_DTYPE_BF16 && in_dtype != HBT_DTYPE_F16 &&
        !(f64 && in_dtype == HBT_DTYPE_F64)) {
        set_error("hbt_grad_local_share_sqnorm: input dtype %d is not F32, BF16 or F16 (or F64 with reduce dtype F64)",
                  in_dtype);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if (reduce_dtype != HBT_DTYPE_F32 && reduce_dtype != HBT_DTYPE_BF16 && reduce_dtype != HBT_DTYPE_F16 && !f64) {
        set_error("hbt_grad_local_share_sqnorm: reduce dtype %d is not F32, BF16, F16 or F64", reduce_dtype);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    ShareRanks ranks{};
    const int elem = dtype_size(in_dtype);
    const int64_t offset = int64_t(rank) * shard_numel;
    int32_t vec_ok = aligned(out, 16);
    for (int q = 0; q < group_size; ++q) {
        if (rank_grads[q] == nullptr && valid_numel > 0) {
            set_error("hbt_grad_local_share_sqnorm: rank %d gradient pointer is null", q);
            return HBT_ERR_INVALID_ARGUMENT;
        }
        ranks.g[q] = static_cast<const uint8_t*>(rank_grads[q]);
        const uintptr_t a = reinterpret_cast<uintptr_t>(ranks.g[q]) + static_cast<uintptr_t>(offset * elem);
        if ((a & static_cast<uintptr_t>(4 * elem - 1)) != 0) vec_ok = 0;
    }
    const int64_t chunk = norm_chunk<float>();
    const int64_t valid_chunks = (valid_numel + chunk - 1) / chunk;
    const int64_t pad_chunks = (shard_numel - valid_numel + chunk - 1) / chunk;
    const int64_t tiles = (shard_numel + kShareTile - 1) / kShareTile;
    const int64_t valid_tiles = (valid_numel + kShareTile - 1) / kShareTile;
    if (tiles == 0) return HBT_OK;
    if (tiles > 0x7FFFFFFFLL) {
        set_error("hbt_grad_local_share_sqnorm: %lld tiles exceed the grid limit", static_cast<long long>(tiles));
        return HBT_ERR_UNSUPPORTED;
    }
    hipStream_t st = as_stream(stream);
    // An exact power of two (or 1) divides as a multiply by its exact reciprocal.
    const float recip = exact_reciprocal(divisor);
    const bool recip_exact = recip != 0.0f;
    const dim3 grid(static_cast<unsigned>(tiles));
#define HBT_TILES(SBYTES, G, R, H, RD)                                                          \
    local_share_tiles_kernel<SBYTES, G, R, H, RD><<<grid, kShareBlock, 0, st>>>(                  \
        ranks, group_size, offset, shard_numel, valid_numel, divisor, recip, vec_ok, out, tile_scratch)
#define HBT_TILES_G(SBYTES, R, H)                                          \
    do {                                                                   \
        switch (group_size) {                                              \
            case 1: HBT_TILES(SBYTES, 1, R, H, HBT_DTYPE_F32); break;      \
            case 2: HBT_TILES(SBYTES, 2, R, H, HBT_DTYPE_F32); break;      \
            case 4: HBT_TILES(SBYTES, 4, R, H, HBT_DTYPE_F32); break;      \
            case 8: HBT_TILES(SBYTES, 8, R, H, HBT_DTYPE_F32); break;      \
            default: HBT_TILES(SBYTES, 0, R, H, HBT_DTYPE_F32); break;     \
        }                                                                  \
    } while (0)
// A 2-byte reduce dtype runs the run-time group size kernel only: the fp32 reduction
// is the configuration the group-size specialisations were tuned for.
#define HBT_TILES_RD(SBYTES, R, H)                                                            \
    do {                                                                                      \
        if (reduce_dtype == HBT_DTYPE_F32) {                                                  \
            HBT_TILES_G(SBYTES, R, H);                                                        \
        } else if (reduce_dtype == HBT_DTYPE_BF16) {                                          \
            HBT_TILES(SBYTES, 0, R, H, HBT_DTYPE_BF16);                                       \
        } else {                                                                              \
            HBT_TILES(SBYTES, 0, R, H, HBT_DTYPE_F16);                                        \
        }                                                                                     \
    } while (0)
#define HBT_TILES64(SBYTES, H)                                                                    \
    local_share_f64_tiles_kernel<SBYTES, H><<<grid, kShareBlock, 0, st>>>(                          \
        ranks, group_size, offset, shard_numel, valid_numel, static_cast<double>(divisor), out, tile_scratch)
    if (f64) {
        if (in_dtype == HBT_DTYPE_F64) HBT_TILES64(8, false);
        else if (in_dtype == HBT_DTYPE_F32) HBT_TILES64(4, false);
        else if (in_dtype == HBT_DTYPE_BF16) HBT_TILES64(2, false);
        else HBT_TILES64(2, true);
    } else if (in_dtype == HBT_DTYPE_F32) {
        if (recip_exact) HBT_TILES_RD(4, true, false); else HBT_TILES_RD(4, false, false);
    } else if (in_dtype == HBT_DTYPE_BF16) {
        if (recip_exact) HBT_TILES_RD(2, true, false); else HBT_TILES_RD(2, false, false);
    } else {
        if (recip_exact) HBT_TILES_RD(2, true, true); else HBT_TILES_RD(2, false, true);
    }
#undef HBT_TILES_RD
#undef HBT_TILES64
#undef HBT_TILES_G
#undef HBT_TILES
    const hipError_t launched = hipGetLastError();
    if (launched != hipSuccess) {
        set_error("hbt_grad_local_share_sqnorm: %s", hipGetErrorString(launched));
        return HBT_ERR_HIP;
    }
    const int64_t chunks = valid_chunks + pad_chunks;
    tile_sums_to_partials_kernel<<<dim3(static_cast<unsigned>(chunks)), kShareBlock, 0, st>>>(
        tile_scratch, valid_tiles, valid_chunks, partials);
    return check_launch("hbt_grad_local_share_sqnorm");
}


int32_t hbt_sgd_step(float* const* params, const void* const* grads, float* const* momentum_buffers,
                     const int64_t* numels, int32_t count, int32_t grad_dtype, float unscale,
                     const float* grad_mul, float weight_decay, float momentum, float one_minus_dampening,
                     float neg_lr, int32_t flags, void* stream) {
    clear_error();
    if (count < 0 || count > kMaxT) {
        set_error("hbt_sgd_step: count must lie in [0, %d], got %d", kMaxT, count);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if (grad_dtype != HBT_DTYPE_F32 && grad_dtype != HBT_DTYPE_BF16) {
        set_error("hbt_sgd_step: gradient dtype %d is not F32 or BF16", grad_dtype);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if ((flags & ~(HBT_SGD_MOMENTUM | HBT_SGD_FIRST_STEP | HBT_SGD_NESTEROV | HBT_SGD_WEIGHT_DECAY)) != 0 ||
        ((flags & (HBT_SGD_FIRST_STEP | HBT_SGD_NESTEROV)) != 0 && (flags & HBT_SGD_MOMENTUM) == 0)) {
        set_error("hbt_sgd_step: bad flags 0x%x", flags);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    const bool with_momentum = (flags & HBT_SGD_MOMENTUM) != 0;
    if (count > 0 && (params == nullptr || grads == nullptr || numels == nullptr ||
                      (with_momentum && momentum_buffers == nullptr))) {
        set_error("hbt_sgd_step: null pointer argument");
        return HBT_ERR_INVALID_ARGUMENT;
    }
    SgdTable tab{};
    tab.count = count;
    const uintptr_t grad_align = grad_dtype == HBT_DTYPE_F32 ? 16 : 8;
    int64_t blocks = 0;
    for (int i = 0; i < count; ++i) {
        if (numels[i] < 0 || (numels[i] > 0 && (params[i] == nullptr || grads[i] == nullptr ||
                                                (with_momentum && momentum_buffers[i] == nullptr)))) {
            set_error("hbt_sgd_step: tensor %d has a bad pointer or numel", i);
            return HBT_ERR_INVALID_ARGUMENT;
        }
        tab.p[i] = params[i];
        tab.g[i] = grads[i];
        tab.buf[i] = with_momentum ? momentum_buffers[i] : nullptr;
        tab.n[i] = numels[i];
        tab.vec_ok[i] = aligned(params[i], 16) && aligned(grads[i], grad_align) &&
                        (!with_momentum || aligned(momentum_buffers[i], 16));
        tab.first_block[i] = blocks;
        blocks += (numels[i] + kAdamTile - 1) / kAdamTile;
    }
    tab.first_block[count] = blocks;
    for (int i = count + 1; i <= kMaxT; ++i) tab.first_block[i] = blocks;
    if (blocks == 0) return HBT_OK;
    if (blocks > 0x7FFFFFFFLL) {
        set_error("hbt_sgd_step: %lld tiles exceed the grid limit", static_cast<long long>(blocks));
        return HBT_ERR_UNSUPPORTED;
    }
    SgdScalars sc{unscale, weight_decay, momentum, one_minus_dampening, neg_lr,
                  (flags & HBT_SGD_WEIGHT_DECAY) != 0, (flags & HBT_SGD_NESTEROV) != 0};
    const int mode = !with_momentum ? kSgdPlain : ((flags & HBT_SGD_FIRST_STEP) ? kSgdFirst : kSgdMomentum);
    const bool scaled = unscale != 1.0f;
    const dim3 grid(static_cast<unsigned>(blocks));
    hipStream_t st = as_stream(stream);
#define HBT_SGD_LAUNCH(GT, SCALED, MODE) \
    sgd_kernel<GT, SCALED, MODE><<<grid, kAdamBlock, 0, st>>>(tab, sc, grad_mul)
#define HBT_SGD_MODES(GT, SCALED)                                          \
    do {                                                                   \
        if (mode == kSgdPlain) HBT_SGD_LAUNCH(GT, SCALED, kSgdPlain);      \
        else if (mode == kSgdFirst) HBT_SGD_LAUNCH(GT, SCALED, kSgdFirst); \
        else HBT_SGD_LAUNCH(GT, SCALED, kSgdMomentum);                     \
    } while (0)
    if (grad_dtype == HBT_DTYPE_F32) {
        if (scaled) HBT_SGD_MODES(float, true); else HBT_SGD_MODES(float, false);
    } else {
        if (scaled) HBT_SGD_MODES(uint16_t, true); else HBT_SGD_MODES(uint16_t, false);
    }
#undef HBT_SGD_MODES
#undef HBT_SGD_LAUNCH
    return check_launch("hbt_sgd_step");
}

}  // extern "C"

