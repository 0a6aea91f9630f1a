// Shared host/device helpers for libhbt.so (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <string>

#include "hbt.h"

namespace hbt {

// ---- error reporting -------------------------------------------------------------
// One message per host thread; set by a failing entry point, read by hbt_last_error().
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

// Returns HBT_ERR_HIP (with a message naming `what`) if a HIP call or the last
// launch failed, else HBT_OK.
int32_t check_hip(hipError_t status, const char* what);
int32_t check_launch(const char* what);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Number of compute units of the current device (cached per device id).
int device_cu_count();

// 1 / divisor when divisor is a power of two whose reciprocal is a normal float, else 0.
// For such a divisor x * (1 / divisor) and x / divisor are the same correctly rounded
// value (both round the same real number), so a division becomes a multiply.
inline float exact_reciprocal(float divisor) {
    int exponent = 0;
    const float mantissa = std::frexp(divisor, &exponent);
    const bool exact = divisor > 0.0f && mantissa == 0.5f && exponent > -125 && exponent < 126;
    return exact ? std::ldexp(1.0f, 1 - exponent) : 0.0f;
}

// ---- launch limits -------------------------------------------------------------------
// A HIP grid dimension holds at most 2^32 - 1 work-items (workgroups x workgroup size),
// so a launch of `threads`-lane workgroups takes at most grid_max_blocks(threads)
// workgroups.  Larger launches are split into consecutive slices of workgroups; slice k
// covers blocks [k * grid_max_blocks, min((k + 1) * grid_max_blocks, blocks)), and each
// kernel adds its slice's first block to blockIdx.x.
constexpr int64_t kGridMaxItems = 0xFFFFFFFFLL;
inline int64_t grid_max_blocks(int threads) { return threads > 0 ? kGridMaxItems / threads : 0; }
inline int64_t grid_slice_count(int64_t blocks, int threads) {
    const int64_t per = grid_max_blocks(threads);
    return (blocks <= 0 || per <= 0) ? 0 : (blocks + per - 1) / per;
}

// Runs launch(first_block, slice_blocks) for every slice of a `blocks`-workgroup grid of
// `threads`-lane workgroups and checks each launch; `who` names the caller in errors.
template <typename Launch>
int32_t launch_sliced(const char* who, int64_t blocks, int threads, Launch&& launch) {
    const int64_t per = grid_max_blocks(threads);
    for (int64_t first = 0; first < blocks; first += per) {
        const int64_t n = blocks - first < per ? blocks - first : per;
        launch(first, dim3(static_cast<unsigned>(n)));
        const int32_t status = check_launch(who);
        if (status != HBT_OK) return status;
    }
    return HBT_OK;
}

// ---- dtype helpers -------------------------------------------------------------------
inline int dtype_size(int32_t dtype) {
    switch (dtype) {
        case HBT_DTYPE_F32: return 4;
        case HBT_DTYPE_BF16: return 2;
        case HBT_DTYPE_F16: return 2;
        case HBT_DTYPE_F64: return 8;
        default: return 0;
    }
}

// bf16 <-> fp32.  Widening is exact (the bf16 bits are the high half of the fp32).
// Narrowing rounds to nearest, ties to even; any NaN becomes the quiet NaN 0x7FC0.
__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
    return __uint_as_float(bits16 << 16);
}

// A select of a constant, not an early return: as a branch it compiles to a per-element
// exec-mask jump, which made the 2-byte norm pass ALU-bound.
__device__ __forceinline__ uint32_t f32_to_bf16(float x) {
    const uint32_t u = __float_as_uint(x);
    const uint32_t rounded = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
    return (u & 0x7FFFFFFFu) > 0x7F800000u ? 0x7FC0u : rounded;
}

// IEEE fp16 <-> fp32 with gfx950's conversion instructions.  Widening (v_cvt_f32_f16) is
// exact, subnormals included; narrowing (v_cvt_f16_f32) rounds to nearest, ties to even,
// overflows to +-inf and keeps fp16 subnormals.  A NaN stays a NaN of the same sign with
// the quiet bit set; its payload is kept (widening) or truncated (narrowing), the rule of
// torch's vectorised CPU conversions (x86 F16C).  torch's scalar CPU loop writes other NaN
// bits, so no NaN encoding is torch's in general.
__device__ __forceinline__ float f16_to_f32(uint32_t bits16) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16)));
}

__device__ __forceinline__ uint32_t f32_to_f16(float x) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
}

// A 2-byte element's fp32 value and back: IEEE fp16 when kHalf, else bf16.
template <bool kHalf>
__device__ __forceinline__ float b16_to_f32(uint32_t bits16) {
    if constexpr (kHalf) return f16_to_f32(bits16);
    return bf16_to_f32(bits16);
}
template <bool kHalf>
__device__ __forceinline__ uint32_t f32_to_b16(float x) {
    if constexpr (kHalf) return f32_to_f16(x);
    return f32_to_bf16(x);
}

// x rounded to dtype RD and widened back to fp32, exactly: unchanged for HBT_DTYPE_F32;
// round to nearest even for HBT_DTYPE_BF16 and HBT_DTYPE_F16 (fp16: overflow to +-inf,
// subnormals kept).  This is the value torch holds after an op whose result dtype is RD
// (the op computed in fp32, then rounded once).  It uses gfx950's conversion
// instructions (v_cvt_pk_bf16_f32, v_cvt_f16_f32), which round to nearest even in the
// IEEE mode these kernels are built for; a NaN stays a NaN (its payload is not
// specified here: every store of a 2-byte value goes through f32_to_b16 above).  The
// empty asm makes the fp32 value opaque to the compiler, so the rounding stays an
// explicit step: otherwise it folds fp32 arithmetic on widened 2-byte operands followed
// by a narrowing into native 2-byte arithmetic (v_add_f16, v_fma_mixlo_f16), whose
// single rounding differs from torch's fp32 operation rounded afterwards.  It costs no
// instruction.
__device__ __forceinline__ float opaque(float x) {
    asm("" : "+v"(x));
    return x;
}
template <int RD>
__device__ __forceinline__ float round_to(float x) {
    if constexpr (RD == HBT_DTYPE_BF16) {
        return static_cast<float>(static_cast<__bf16>(opaque(x)));
    } else if constexpr (RD == HBT_DTYPE_F16) {
        return static_cast<float>(static_cast<_Float16>(opaque(x)));
    } else {
        return x;
    }
}

// Two fp32 values rounded to the 2-byte dtype RD (nearest even) and packed low half first by
// one packed conversion: the bits f32_to_b16 gives for each, except that a bf16 NaN keeps the
// conversion's encoding (pack_rounded and store_vec write 0x7FC0 instead).
template <int RD>
__device__ __forceinline__ uint32_t pack2_rounded(float a, float b) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    if constexpr (RD == HBT_DTYPE_BF16) {
        typedef __bf16 r2 __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{opaque(a), opaque(b)}, r2));
    } else {
        static_assert(RD == HBT_DTYPE_F16, "2-byte dtypes are bf16 and fp16");
        typedef _Float16 r2 __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{opaque(a), opaque(b)}, r2));
    }
}

// 2N fp32 values rounded to the 2-byte dtype RD and packed into N dwords, a bf16 NaN as
// 0x7FC0: f32_to_b16's bits for each, in N conversions and 2N compares, where f32_to_b16
// takes about 7 operations per element.
template <int RD, int N>
__device__ __forceinline__ void pack_rounded(const float (&y)[2 * N], uint32_t (&o)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) o[i] = pack2_rounded<RD>(y[2 * i], y[2 * i + 1]);
    if constexpr (RD == HBT_DTYPE_BF16) {
        bool nan = false;
#pragma unroll
        for (int c = 0; c < 2 * N; ++c) nan = nan || y[c] != y[c];
        if (nan) {
#pragma unroll
            for (int i = 0; i < N; ++i) {
                if (y[2 * i] != y[2 * i]) o[i] = (o[i] & 0xFFFF0000u) | 0x7FC0u;
                if (y[2 * i + 1] != y[2 * i + 1]) o[i] = (o[i] & 0xFFFFu) | 0x7FC00000u;
            }
        }
    }
}

// The dtype code of SB-byte elements (a 2-byte element being fp16 when H, else bf16).
template <int SB, bool H>
constexpr int dtype_of() {
    return SB == 4 ? HBT_DTYPE_F32 : (H ? HBT_DTYPE_F16 : HBT_DTYPE_BF16);
}

// Element i of an array of B-byte floats (float64, float32, or bf16 / fp16 when H)
// widened exactly to double: Tensor.to(float64).
template <int B, bool H>
__device__ __forceinline__ double widen_f64(const unsigned char* p, int64_t i) {
    if constexpr (B == 8) return reinterpret_cast<const double*>(p)[i];
    else if constexpr (B == 4) return static_cast<double>(reinterpret_cast<const float*>(p)[i]);
    else return static_cast<double>(b16_to_f32<H>(reinterpret_cast<const uint16_t*>(p)[i]));
}

// ---- fixed-order reductions ----------------------------------------------------------
// A double moved between lanes of each 16-lane row by the DPP control kCtrl (a row
// rotation or a quad permutation).
template <int kCtrl>
__device__ __forceinline__ double dpp_move(double x) {
    const uint64_t b = static_cast<uint64_t>(__double_as_longlong(x));
    const uint32_t lo = __builtin_amdgcn_mov_dpp(static_cast<int>(static_cast<uint32_t>(b)), kCtrl, 0xF, 0xF, false);
    const uint32_t hi = __builtin_amdgcn_mov_dpp(static_cast<int>(static_cast<uint32_t>(b >> 32)), kCtrl, 0xF, 0xF, false);
    return __longlong_as_double(static_cast<long long>((uint64_t(hi) << 32) | lo));
}
// The double of lane ^ M, M = 32 or 16, by the gfx950 half-wave / row swaps: a swap of x
// with itself leaves the upper half's (odd rows') values in the second result and the
// lower half's (even rows') in the first; a lane takes the half it is not in.
template <int M>
__device__ __forceinline__ double swap_move(double x) {
    const uint64_t b = static_cast<uint64_t>(__double_as_longlong(x));
    const uint32_t lo = static_cast<uint32_t>(b), hi = static_cast<uint32_t>(b >> 32);
    const bool upper = (__lane_id() & M) != 0;
    uint32_t rlo, rhi;
    if constexpr (M == 32) {
        const auto l = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
        const auto h = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
        rlo = upper ? l[0] : l[1];
        rhi = upper ? h[0] : h[1];
    } else {
        static_assert(M == 16, "row swaps exchange 32- or 16-lane groups");
        const auto l = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
        const auto h = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
        rlo = upper ? l[0] : l[1];
        rhi = upper ? h[0] : h[1];
    }
    return __longlong_as_double(static_cast<long long>((uint64_t(rhi) << 32) | rlo));
}

// Butterfly over the 64 lanes of a wavefront: x += x[lane ^ m] for m = 32, 16, ..., 1;
// every lane ends with the same total and the pairing order is fixed, so the result is
// reproducible bit for bit.  The exchanges are VALU moves, not LDS permutes: m = 32 and 16
// by the half-wave and row swaps (lane ^ m exactly); m = 8, 4, 2, 1 by row rotations and
// quad permutations, which read lane i ^ m ^ (a combination of the bits above m).  Those
// bits are already summed over at that stage (a + b == b + a), so every such lane holds
// lane i ^ m's value and each lane's sum is bitwise the exchange butterfly's.
__device__ __forceinline__ double wave_sum(double x) {
    x += swap_move<32>(x);
    x += swap_move<16>(x);
    x += dpp_move<0x128>(x);  // row_ror:8
    x += dpp_move<0x124>(x);  // row_ror:4
    x += dpp_move<0x4E>(x);   // quad_perm [2, 3, 0, 1]
    x += dpp_move<0xB1>(x);   // quad_perm [1, 0, 3, 2]
    return x;
}

// Sum over a block of BLOCK threads (BLOCK a multiple of 64, at most 1024).  Wave
// totals are combined by wave 0 in wave order.  Result valid in thread 0.
template <int BLOCK>
__device__ __forceinline__ double block_sum(double x) {
    constexpr int kWaves = BLOCK / 64;
    __shared__ double wave_totals[kWaves];
    x = wave_sum(x);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    if (lane == 0) wave_totals[wave] = x;
    __syncthreads();
    double total = 0.0;
    if (threadIdx.x == 0) {
#pragma unroll
        for (int w = 0; w < kWaves; ++w) total += wave_totals[w];
    }
    return total;
}

}  // namespace hbt
