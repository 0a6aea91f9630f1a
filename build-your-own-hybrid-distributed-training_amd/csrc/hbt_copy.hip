// Interval gather-copy (gfx950).
//
// One launch moves any number of [src, src + n) -> [dst, dst + n) intervals.  Each
// interval is cut into chunks of 64 x 16 bytes of source (256 elements of a 4-byte
// source, 512 of a 2-byte one); one workgroup owns one chunk and finds its interval by
// a binary search over the records' first_chunk column.  Inside a chunk each lane moves
// units of 16 / max(source, destination element bytes) elements, consecutive lanes
// taking consecutive units, so every load and store instruction of a wave covers one
// contiguous span.
//
// Two kernels share that layout.  copy_aligned_kernel serves plans whose records all
// start on aligned addresses (the host certifies this): one aligned load and one aligned
// store per unit.  copy_kernel serves any plan: the destination is written with aligned
// stores after an element-wise head, and the source is read with aligned loads of the
// unit's width and shifted into place with v_alignbyte, so intervals at any element
// offset stream at full width.  A load never touches an aligned block that holds no byte
// of the source interval.
#include "hbt_common.hpp"

namespace hbt {
namespace {

// One wavefront per workgroup reading 16 bytes of source per lane: a workgroup reads
// 1 KB and retires, the shape that streamed fastest against 512 B or 2 KB per
// workgroup and against 256-thread workgroups walking larger chunks.
constexpr int kCopyBlock = 64;
// Non-temporal loads and stores: every byte is moved once.
constexpr bool kCopyNT = true;

// A vector of NW dwords (NW = 2 or 4).
template <int NW>
struct Vec {
    typedef uint32_t type __attribute__((ext_vector_type(NW)));
};

// The copy kernel reads its addresses from a table in device memory, so the compiler
// cannot tell which address space they point into and would issue flat loads and
// stores.  These views name global memory (address space 1): global_load/global_store
// instructions, which wait on the vector counter alone.
typedef __attribute__((address_space(1))) uint8_t gbyte;

// Aligned vector load/store of NW dwords, non-temporal when kCopyNT: every byte is moved
// exactly once.
template <int NW>
__device__ __forceinline__ typename Vec<NW>::type ldg(const gbyte* p) {
    typedef typename Vec<NW>::type V;
    typedef __attribute__((address_space(1))) const V GV;
    if constexpr (kCopyNT) return __builtin_nontemporal_load(reinterpret_cast<GV*>(p));
    return *reinterpret_cast<GV*>(p);
}
template <int NW>
__device__ __forceinline__ void stg(gbyte* p, typename Vec<NW>::type x) {
    typedef typename Vec<NW>::type V;
    typedef __attribute__((address_space(1))) V GV;
    if constexpr (kCopyNT) {
        __builtin_nontemporal_store(x, reinterpret_cast<GV*>(p));
    } else {
        *reinterpret_cast<GV*>(p) = x;
    }
}

// A unit's source bytes as loaded: one aligned block, plus the next one when the
// source is misaligned by k = s mod 4*NW bytes (k is uniform across the wave).  The
// second block holds source bytes s + 4*NW - 1 and earlier ones only up to the block
// boundary, so it lies inside the source's page.
template <int NW>
struct Raw {
    typename Vec<NW>::type x, y;
};
template <int NW>
__device__ __forceinline__ void load_raw(const gbyte* s, uint32_t k, Raw<NW>& r) {
    static_assert(NW == 2 || NW == 4, "units are 8 or 16 bytes");
    const gbyte* a = s - k;
    r.x = ldg<NW>(a);
    if (k != 0) r.y = ldg<NW>(a + 4 * NW);
}
// Shifts a loaded unit into place with v_alignbyte.
template <int NW>
__device__ __forceinline__ void align_raw(const Raw<NW>& raw, uint32_t k, uint32_t (&out)[NW]) {
    if (k == 0) {
#pragma unroll
        for (int i = 0; i < NW; ++i) out[i] = raw.x[i];
        return;
    }
    uint32_t w[2 * NW];
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        w[i] = raw.x[i];
        w[NW + i] = raw.y[i];
    }
    const uint32_t r = k & 3u;
    const uint32_t q = k >> 2;  // whole dwords to skip, < NW
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        // Select w[i + q] and w[i + q + 1] with q uniform; unrolled over q's range.
        uint32_t lo = w[i], hi = w[i + 1];
#pragma unroll
        for (int j = 1; j < NW; ++j) {
            if (q == static_cast<uint32_t>(j)) {
                lo = w[i + j];
                hi = w[i + j + 1];
            }
        }
        out[i] = __builtin_amdgcn_alignbyte(hi, lo, r);
    }
}

// Element semantics.  SB/DB are source/destination element bytes; a 2-byte element is
// bf16, or IEEE fp16 when H is set (a conversion never mixes the two).  Same-size COPY
// is a bit copy; 4->2 narrows fp32 (round to nearest even), 2->4 widens exactly; DIVIDE
// goes through fp32 (true division) and rounds to the destination type.
template <int SB, bool H>
__device__ __forceinline__ float elem_to_f32(uint32_t bits) {
    if constexpr (SB == 4) return __uint_as_float(bits);
    return b16_to_f32<H>(bits);
}
template <int DB, bool H>
__device__ __forceinline__ uint32_t f32_to_elem(float x) {
    if constexpr (DB == 4) return __float_as_uint(x);
    return f32_to_b16<H>(x);
}
// kOpScale: HBT_COPY_OP_DIVIDE by a power of two, run as a multiply by its exact
// reciprocal (passed in place of the divisor); the bits are those of the division.
constexpr int kOpScale = 2;
template <int SB, int OP, bool H>
__device__ __forceinline__ float convert_value(uint32_t bits, float divisor) {
    float x = elem_to_f32<SB, H>(bits);
    if constexpr (OP == HBT_COPY_OP_DIVIDE) x = x / divisor;
    if constexpr (OP == kOpScale) x = x * divisor;
    return x;
}
template <int SB, int DB, int OP, bool H>
__device__ __forceinline__ uint32_t convert(uint32_t bits, float divisor) {
    if constexpr (SB == DB && OP == HBT_COPY_OP_COPY) return bits;
    return f32_to_elem<DB, H>(convert_value<SB, OP, H>(bits, divisor));
}
// Whether a copy rounds fp32 values to a 2-byte destination (a narrowing, or arithmetic on
// 2-byte elements): the vector paths then round two values per packed conversion.
template <int SB, int DB, int OP>
constexpr bool rounds_to_b16() { return DB == 2 && !(SB == 2 && OP == HBT_COPY_OP_COPY); }

template <int EB>
__device__ __forceinline__ uint32_t load_elem(const gbyte* p) {
    typedef __attribute__((address_space(1))) const uint32_t G32;
    typedef __attribute__((address_space(1))) const uint16_t G16;
    if constexpr (EB == 4) return *reinterpret_cast<G32*>(p);
    return *reinterpret_cast<G16*>(p);
}
template <int EB>
__device__ __forceinline__ void store_elem(gbyte* p, uint32_t bits) {
    typedef __attribute__((address_space(1))) uint32_t G32;
    typedef __attribute__((address_space(1))) uint16_t G16;
    if constexpr (EB == 4) {
        *reinterpret_cast<G32*>(p) = bits;
    } else {
        *reinterpret_cast<G16*>(p) = static_cast<uint16_t>(bits);
    }
}

// Elements per lane unit: one 16-byte access on the wider side of the copy.
template <int SB, int DB>
constexpr int unit_elems() { return 16 / (SB > DB ? SB : DB); }
// Elements per chunk (per workgroup): 16 bytes of source per lane, 32 when the
// destination is wider.  A widening chunk writes more than it reads, and its stores do
// not hold the workgroup, so with 1 KB of source the workgroups retired faster than
// their writes drained; same-size and narrowing copies keep 1 KB.
template <int SB, int DB>
constexpr int64_t chunk_elems() { return int64_t(kCopyBlock) * 16 / SB * (SB < DB ? 2 : 1); }

// Unpack the U elements held in `words` (SB bytes each) into element bit patterns.
template <int SB, int U>
__device__ __forceinline__ void unpack_unit(const uint32_t (&words)[U * SB / 4], uint32_t (&e)[U]) {
    if constexpr (SB == 4) {
#pragma unroll
        for (int i = 0; i < U; ++i) e[i] = words[i];
    } else {
#pragma unroll
        for (int i = 0; i < U / 2; ++i) {
            e[2 * i] = words[i] & 0xFFFFu;
            e[2 * i + 1] = words[i] >> 16;
        }
    }
}
template <int DB, int U>
__device__ __forceinline__ void pack_unit_store(gbyte* d, const uint32_t (&e)[U]) {
    constexpr int NW = U * DB / 4;
    typename Vec<NW>::type x;
    if constexpr (DB == 4) {
#pragma unroll
        for (int i = 0; i < U; ++i) x[i] = e[i];
    } else {
#pragma unroll
        for (int i = 0; i < U / 2; ++i) x[i] = e[2 * i] | (e[2 * i + 1] << 16);
    }
    stg<NW>(d, x);
}

// Index of the record that owns `chunk`: the last record whose first_chunk <= chunk
// (the host drops records with no chunks, so first_chunk strictly increases).  The
// search runs on the scalar unit: its loads hit the scalar cache and do not queue behind
// the vector traffic of the waves in flight (a wave-wide search over vector loads waits
// behind that traffic and was slower).  With
// hints (the table followed by hints[j] = the record owning chunk j * kHintStride) the
// search starts at the hinted record and steps forward, at most as many records as
// start inside one hint stride; without them it bisects the whole table, log2(count)
// dependent loads before the workgroup's first data load.
constexpr int kHintShift = 8;  // one hint per 256 chunks
__device__ __forceinline__ int64_t owning_record(const int64_t* __restrict__ table, int64_t count,
                                                 int64_t chunk, const int64_t* __restrict__ hints) {
    if (hints != nullptr) {
        int64_t r = hints[chunk >> kHintShift];
        r = r < 0 ? 0 : (r < count ? r : count - 1);  // a wrong hint stays inside the table
        while (r + 1 < count && table[4 * (r + 1) + 3] <= chunk) ++r;
        return r;
    }
    int64_t lo = 0, hi = count - 1;
    while (lo < hi) {
        const int64_t mid = (lo + hi + 1) >> 1;
        if (table[4 * mid + 3] <= chunk) {
            lo = mid;
        } else {
            hi = mid - 1;
        }
    }
    return lo;
}

template <int SB, int DB, int OP, bool H>
__global__ __launch_bounds__(kCopyBlock) void copy_kernel(const int64_t* __restrict__ table,
                                                          int64_t count, float divisor, int64_t chunk_base,
                                                          const int64_t* __restrict__ hints) {
    static_assert(kCopyBlock == 64, "a workgroup is one wave; its chunk is whole wave-wide spans of 16-byte source loads");
    const int64_t chunk = chunk_base + static_cast<int64_t>(blockIdx.x);
    const int64_t* rec = table + 4 * owning_record(table, count, chunk, hints);
    const gbyte* src = reinterpret_cast<const gbyte*>(static_cast<uintptr_t>(rec[0]));
    gbyte* dst = reinterpret_cast<gbyte*>(static_cast<uintptr_t>(rec[1]));
    const int64_t n = rec[2];
    constexpr int64_t kChunk = chunk_elems<SB, DB>();
    const int64_t e0 = (chunk - rec[3]) * kChunk;
    const int64_t len = (n - e0) < kChunk ? (n - e0) : kChunk;

    gbyte* d = dst + e0 * DB;
    const gbyte* s = src != nullptr ? src + e0 * SB : nullptr;
    constexpr int U = unit_elems<SB, DB>();
    constexpr int kSrcWords = U * SB / 4;
    constexpr int kPerLane = static_cast<int>(kChunk / U / kCopyBlock);
    static_assert(kChunk == int64_t(kPerLane) * kCopyBlock * U, "a chunk is whole units on every lane");

    // Head: elements until the destination is 16-byte aligned.
    int64_t head = static_cast<int64_t>(((16u - (static_cast<uint32_t>(reinterpret_cast<uintptr_t>(d)) & 15u)) & 15u) / DB);
    if (head > len) head = len;
    const int64_t units = (len - head) / U;
    const int64_t tail_begin = head + units * U;

    if (threadIdx.x < head) {
        const int64_t e = threadIdx.x;
        const uint32_t bits = s != nullptr ? convert<SB, DB, OP, H>(load_elem<SB>(s + e * SB), divisor) : 0u;
        store_elem<DB>(d + e * DB, bits);
    }
    if (threadIdx.x < len - tail_begin) {
        const int64_t e = tail_begin + threadIdx.x;
        const uint32_t bits = s != nullptr ? convert<SB, DB, OP, H>(load_elem<SB>(s + e * SB), divisor) : 0u;
        store_elem<DB>(d + e * DB, bits);
    }

    // Units per lane: kPerLane (2 for bf16 -> fp32, else 1).  Every unit's loads are
    // issued before the first store, so a workgroup pays one memory round trip.
    gbyte* dbody = d + head * DB;
    if (s == nullptr) {
        uint32_t zero[U];
#pragma unroll
        for (int i = 0; i < U; ++i) zero[i] = 0u;
#pragma unroll
        for (int j = 0; j < kPerLane; ++j) {
            const int64_t u = threadIdx.x + j * kCopyBlock;
            if (u < units) pack_unit_store<DB, U>(dbody + u * U * DB, zero);
        }
        return;
    }
    const gbyte* sbody = s + head * SB;
    const uint32_t k = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(sbody)) & (4u * kSrcWords - 1u);
    Raw<kSrcWords> raw[kPerLane];
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
        const int64_t u = threadIdx.x + j * kCopyBlock;
        if (u < units) load_raw<kSrcWords>(sbody + u * U * SB, k, raw[j]);
    }
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
        const int64_t u = threadIdx.x + j * kCopyBlock;
        if (u < units) {
            uint32_t words[kSrcWords];
            align_raw<kSrcWords>(raw[j], k, words);
            uint32_t e[U];
            unpack_unit<SB, U>(words, e);
#pragma unroll
            for (int i = 0; i < U; ++i) e[i] = convert<SB, DB, OP, H>(e[i], divisor);
            pack_unit_store<DB, U>(dbody + u * U * DB, e);
        }
    }
}

// Aligned-record copy: every record's destination is 16-byte aligned and its source is
// aligned to the unit's source width (the host certifies this for the whole plan), so a
// lane moves its unit with one aligned load and one aligned store.  A chunk's units past
// the record's end are masked off; a record whose length is not a whole number of units
// finishes with an element loop in its last chunk.
template <int SB, int DB, int OP, bool H>
__global__ __launch_bounds__(kCopyBlock) void copy_aligned_kernel(const int64_t* __restrict__ table,
                                                                  int64_t count, float divisor, int64_t chunk_base,
                                                                  const int64_t* __restrict__ hints) {
    constexpr int U = unit_elems<SB, DB>();
    constexpr int kSrcWords = U * SB / 4;
    constexpr int64_t kChunk = chunk_elems<SB, DB>();
    constexpr int kPerLane = static_cast<int>(kChunk / U / kCopyBlock);
    static_assert(kChunk == int64_t(kPerLane) * kCopyBlock * U, "a chunk is whole units on every lane");
    const int64_t chunk = chunk_base + static_cast<int64_t>(blockIdx.x);
    const int64_t* rec = table + 4 * owning_record(table, count, chunk, hints);
    const int64_t e0 = (chunk - rec[3]) * kChunk;
    const int64_t n = rec[2];
    const int64_t len = (n - e0) < kChunk ? (n - e0) : kChunk;
    const int64_t units = len / U;
    const gbyte* s = reinterpret_cast<const gbyte*>(static_cast<uintptr_t>(rec[0]));
    gbyte* d = reinterpret_cast<gbyte*>(static_cast<uintptr_t>(rec[1])) + e0 * DB;
    if (s == nullptr) {
        uint32_t zero[U];
#pragma unroll
        for (int i = 0; i < U; ++i) zero[i] = 0u;
#pragma unroll
        for (int j = 0; j < kPerLane; ++j) {
            const int64_t u = threadIdx.x + j * kCopyBlock;
            if (u < units) pack_unit_store<DB, U>(d + u * U * DB, zero);
        }
        if (threadIdx.x < len - units * U) store_elem<DB>(d + (units * U + threadIdx.x) * DB, 0u);
        return;
    }
    s += e0 * SB;
    typename Vec<kSrcWords>::type x[kPerLane];
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
        const int64_t u = threadIdx.x + j * kCopyBlock;
        if (u < units) x[j] = ldg<kSrcWords>(s + u * U * SB);
    }
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
        const int64_t u = threadIdx.x + j * kCopyBlock;
        if (u < units) {
            uint32_t words[kSrcWords];
#pragma unroll
            for (int i = 0; i < kSrcWords; ++i) words[i] = x[j][i];
            uint32_t e[U];
            unpack_unit<SB, U>(words, e);
            if constexpr (rounds_to_b16<SB, DB, OP>()) {
                // Two values per packed conversion, each the bits f32_to_b16 gives.
                float f[U];
#pragma unroll
                for (int i = 0; i < U; ++i) f[i] = convert_value<SB, OP, H>(e[i], divisor);
                uint32_t w[U / 2];
                pack_rounded<H ? HBT_DTYPE_F16 : HBT_DTYPE_BF16, U / 2>(f, w);
                typename Vec<U / 2>::type o;
#pragma unroll
                for (int i = 0; i < U / 2; ++i) o[i] = w[i];
                stg<U / 2>(d + u * U * DB, o);
            } else {
#pragma unroll
                for (int i = 0; i < U; ++i) e[i] = convert<SB, DB, OP, H>(e[i], divisor);
                pack_unit_store<DB, U>(d + u * U * DB, e);
            }
        }
    }
    if (threadIdx.x < len - units * U) {
        const int64_t e = units * U + threadIdx.x;
        store_elem<DB>(d + e * DB, convert<SB, DB, OP, H>(load_elem<SB>(s + e * SB), divisor));
    }
}

// ---- conversions through double ---------------------------------------------------------
// The dtype pairs the kernels above do not move: float64 to or from another dtype, float64
// divided by the AVG divisor (the pre-divide of float64 DDP buckets), and bf16 <-> fp16.
// Each value widens exactly to double and narrows as torch's Tensor.to does: kept for a
// float64 destination, else to fp32 with one rounding to nearest even, then, for a 2-byte
// destination, to that dtype (double -> fp32 -> bf16/fp16, as c10's conversions go;
// bf16 <-> fp16 through the exact fp32 value).  DIVIDE divides the double by the divisor,
// correctly rounded, as torch's div_ on a float64 tensor does; a power-of-two divisor runs
// as a multiply by its exact reciprocal (kOpScale), with the same bits.  A chunk is 1 KB
// of source, as in the kernels above.
template <int D>
constexpr int elem_bytes() { return D == HBT_DTYPE_F64 ? 8 : (D == HBT_DTYPE_F32 ? 4 : 2); }

template <int D>
__device__ __forceinline__ double widen_elem(const gbyte* p) {
    typedef __attribute__((address_space(1))) const double G64;
    if constexpr (D == HBT_DTYPE_F64) return *reinterpret_cast<G64*>(p);
    else if constexpr (D == HBT_DTYPE_F32) return static_cast<double>(__uint_as_float(load_elem<4>(p)));
    else return static_cast<double>(b16_to_f32<D == HBT_DTYPE_F16>(load_elem<2>(p)));
}
template <int D>
__device__ __forceinline__ void narrow_store(gbyte* p, double x) {
    typedef __attribute__((address_space(1))) double G64;
    if constexpr (D == HBT_DTYPE_F64) {
        *reinterpret_cast<G64*>(p) = x;
    } else if constexpr (D == HBT_DTYPE_F32) {
        store_elem<4>(p, __float_as_uint(static_cast<float>(x)));
    } else {
        store_elem<2>(p, f32_to_b16<D == HBT_DTYPE_F16>(static_cast<float>(x)));
    }
}
template <int OP>
__device__ __forceinline__ double apply_op(double x, double divisor) {
    if constexpr (OP == HBT_COPY_OP_DIVIDE) return x / divisor;
    if constexpr (OP == kOpScale) return x * divisor;
    return x;
}

// NW dwords at p (4 * NW bytes, aligned to that), non-temporal when kCopyNT.
template <int NW>
__device__ __forceinline__ void load_words(const gbyte* p, uint32_t (&w)[NW]) {
    if constexpr (NW == 1) {
        typedef __attribute__((address_space(1))) const uint32_t G32;
        if constexpr (kCopyNT) w[0] = __builtin_nontemporal_load(reinterpret_cast<G32*>(p));
        else w[0] = *reinterpret_cast<G32*>(p);
    } else {
        const typename Vec<NW>::type v = ldg<NW>(p);
#pragma unroll
        for (int i = 0; i < NW; ++i) w[i] = v[i];
    }
}
template <int NW>
__device__ __forceinline__ void store_words(gbyte* p, const uint32_t (&w)[NW]) {
    if constexpr (NW == 1) {
        typedef __attribute__((address_space(1))) uint32_t G32;
        if constexpr (kCopyNT) __builtin_nontemporal_store(w[0], reinterpret_cast<G32*>(p));
        else *reinterpret_cast<G32*>(p) = w[0];
    } else {
        typename Vec<NW>::type v;
#pragma unroll
        for (int i = 0; i < NW; ++i) v[i] = w[i];
        stg<NW>(p, v);
    }
}
// U elements of dtype D held in dwords, to and from their double values (widening exact,
// narrowing as narrow_store narrows).
template <int D, int U>
__device__ __forceinline__ void words_to_f64(const uint32_t (&w)[U * elem_bytes<D>() / 4], double (&x)[U]) {
    if constexpr (D == HBT_DTYPE_F64) {
#pragma unroll
        for (int i = 0; i < U; ++i) x[i] = __hiloint2double(static_cast<int>(w[2 * i + 1]), static_cast<int>(w[2 * i]));
    } else if constexpr (D == HBT_DTYPE_F32) {
#pragma unroll
        for (int i = 0; i < U; ++i) x[i] = static_cast<double>(__uint_as_float(w[i]));
    } else {
#pragma unroll
        for (int i = 0; i < U / 2; ++i) {
            x[2 * i] = static_cast<double>(b16_to_f32<D == HBT_DTYPE_F16>(w[i] & 0xFFFFu));
            x[2 * i + 1] = static_cast<double>(b16_to_f32<D == HBT_DTYPE_F16>(w[i] >> 16));
        }
    }
}
template <int D, int U>
__device__ __forceinline__ void f64_to_words(const double (&x)[U], uint32_t (&w)[U * elem_bytes<D>() / 4]) {
    if constexpr (D == HBT_DTYPE_F64) {
#pragma unroll
        for (int i = 0; i < U; ++i) {
            w[2 * i] = static_cast<uint32_t>(__double2loint(x[i]));
            w[2 * i + 1] = static_cast<uint32_t>(__double2hiint(x[i]));
        }
    } else if constexpr (D == HBT_DTYPE_F32) {
#pragma unroll
        for (int i = 0; i < U; ++i) w[i] = __float_as_uint(static_cast<float>(x[i]));
    } else {
#pragma unroll
        for (int i = 0; i < U / 2; ++i)
            w[i] = f32_to_b16<D == HBT_DTYPE_F16>(static_cast<float>(x[2 * i])) |
                   (f32_to_b16<D == HBT_DTYPE_F16>(static_cast<float>(x[2 * i + 1])) << 16);
    }
}

// Any plan: lane l converts elements l, l + 64, ... of its chunk, so every load and store
// instruction of the wave covers one contiguous span.
template <int SD, int DD, int OP>
__global__ __launch_bounds__(kCopyBlock) void convert_kernel(const int64_t* __restrict__ table, int64_t count,
                                                             double divisor, int64_t chunk_base,
                                                             const int64_t* __restrict__ hints) {
    constexpr int64_t SB = elem_bytes<SD>();
    constexpr int64_t DB = elem_bytes<DD>();
    constexpr int64_t kChunk = chunk_elems<SB, DB>();
    const int64_t chunk = chunk_base + static_cast<int64_t>(blockIdx.x);
    const int64_t* rec = table + 4 * owning_record(table, count, chunk, hints);
    const int64_t e0 = (chunk - rec[3]) * kChunk;
    const int64_t n = rec[2];
    const int64_t len = (n - e0) < kChunk ? (n - e0) : kChunk;
    const gbyte* s = reinterpret_cast<const gbyte*>(static_cast<uintptr_t>(rec[0]));
    gbyte* d = reinterpret_cast<gbyte*>(static_cast<uintptr_t>(rec[1])) + e0 * DB;
    if (s != nullptr) s += e0 * SB;
    for (int64_t i = threadIdx.x; i < len; i += kCopyBlock) {
        narrow_store<DD>(d + i * DB, s != nullptr ? apply_op<OP>(widen_elem<SD>(s + i * SB), divisor) : 0.0);
    }
}

// Aligned plans (every destination 16-byte aligned, every source aligned to its unit): a
// lane moves units of U = 16 / max(source, destination bytes) elements, one access of
// U * bytes on each side (16 on the wider side; 8 or 4 on the narrower one), consecutive
// lanes on consecutive units; a 1 KB-of-source chunk is kPerLane units per lane (1 for a
// float64 source; a widening chunk is 2 KB of source, 4 or 8 units per lane), all loaded
// before the first store.
// The bits are convert_kernel's.
template <int SD, int DD, int OP>
__global__ __launch_bounds__(kCopyBlock) void convert_aligned_kernel(const int64_t* __restrict__ table,
                                                                     int64_t count, double divisor,
                                                                     int64_t chunk_base,
                                                                     const int64_t* __restrict__ hints) {
    constexpr int SB = elem_bytes<SD>();
    constexpr int DB = elem_bytes<DD>();
    constexpr int U = 16 / (SB > DB ? SB : DB);
    constexpr int SW = U * SB / 4;
    constexpr int DW = U * DB / 4;
    constexpr int64_t kChunk = chunk_elems<SB, DB>();
    constexpr int kPerLane = static_cast<int>(kChunk / (int64_t(kCopyBlock) * U));
    static_assert(kChunk == int64_t(kPerLane) * kCopyBlock * U, "a chunk is whole units on every lane");
    const int64_t chunk = chunk_base + static_cast<int64_t>(blockIdx.x);
    const int64_t* rec = table + 4 * owning_record(table, count, chunk, hints);
    const int64_t e0 = (chunk - rec[3]) * kChunk;
    const int64_t n = rec[2];
    const int64_t len = (n - e0) < kChunk ? (n - e0) : kChunk;
    const int64_t units = len / U;
    const gbyte* s = reinterpret_cast<const gbyte*>(static_cast<uintptr_t>(rec[0]));
    gbyte* d = reinterpret_cast<gbyte*>(static_cast<uintptr_t>(rec[1])) + e0 * DB;
    if (s == nullptr) {
        uint32_t zero[DW];
#pragma unroll
        for (int i = 0; i < DW; ++i) zero[i] = 0u;
#pragma unroll
        for (int j = 0; j < kPerLane; ++j) {
            const int64_t u = threadIdx.x + j * kCopyBlock;
            if (u < units) store_words<DW>(d + u * U * DB, zero);
        }
        if (threadIdx.x < len - units * U) narrow_store<DD>(d + (units * U + threadIdx.x) * DB, 0.0);
        return;
    }
    s += e0 * SB;
    uint32_t w[kPerLane][SW];
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
        const int64_t u = threadIdx.x + j * kCopyBlock;
        if (u < units) load_words<SW>(s + u * U * SB, w[j]);
    }
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
        const int64_t u = threadIdx.x + j * kCopyBlock;
        if (u < units) {
            double x[U];
            words_to_f64<SD, U>(w[j], x);
#pragma unroll
            for (int i = 0; i < U; ++i) x[i] = apply_op<OP>(x[i], divisor);
            uint32_t o[DW];
            f64_to_words<DD, U>(x, o);
            store_words<DW>(d + u * U * DB, o);
        }
    }
    if (threadIdx.x < len - units * U) {
        const int64_t e = units * U + threadIdx.x;
        narrow_store<DD>(d + e * DB, apply_op<OP>(widen_elem<SD>(s + e * SB), divisor));
    }
}

template <int OP>
int32_t launch_convert(int32_t src_dtype, int32_t dst_dtype, const int64_t* table, int64_t count, int64_t chunks,
                       double divisor, bool aligned, const int64_t* hints, hipStream_t st) {
    return launch_sliced("hbt_copy_intervals", chunks, kCopyBlock, [&](int64_t first, dim3 grid) {
#define HBT_CVT(SD, DD)                                                                                        \
    do {                                                                                                       \
        if (aligned) convert_aligned_kernel<SD, DD, OP><<<grid, kCopyBlock, 0, st>>>(table, count, divisor, first, hints); \
        else convert_kernel<SD, DD, OP><<<grid, kCopyBlock, 0, st>>>(table, count, divisor, first, hints);    \
    } while (0)
        if constexpr (OP != HBT_COPY_OP_COPY) {
            HBT_CVT(HBT_DTYPE_F64, HBT_DTYPE_F64);  // the only division through double
        } else {
#define HBT_CVT_TO(SD)                                                                                   \
    do {                                                                                                 \
        if (dst_dtype == HBT_DTYPE_F64) HBT_CVT(SD, HBT_DTYPE_F64);                                      \
        else if (dst_dtype == HBT_DTYPE_F32) HBT_CVT(SD, HBT_DTYPE_F32);                                 \
        else if (dst_dtype == HBT_DTYPE_BF16) HBT_CVT(SD, HBT_DTYPE_BF16);                               \
        else HBT_CVT(SD, HBT_DTYPE_F16);                                                                 \
    } while (0)
            if (src_dtype == HBT_DTYPE_F64) HBT_CVT_TO(HBT_DTYPE_F64);
            else if (src_dtype == HBT_DTYPE_F32) HBT_CVT_TO(HBT_DTYPE_F32);
            else if (src_dtype == HBT_DTYPE_BF16) HBT_CVT_TO(HBT_DTYPE_BF16);
            else HBT_CVT_TO(HBT_DTYPE_F16);
#undef HBT_CVT_TO
        }
#undef HBT_CVT
    });
}

template <int SB, int DB, int OP, bool H = false>
int32_t launch_copy(const int64_t* table, int64_t count, int64_t chunks, float divisor, bool aligned,
                    const int64_t* hints, hipStream_t s) {
    return launch_sliced("hbt_copy_intervals", chunks, kCopyBlock, [&](int64_t first, dim3 grid) {
        if (aligned) {
            copy_aligned_kernel<SB, DB, OP, H><<<grid, kCopyBlock, 0, s>>>(table, count, divisor, first, hints);
        } else {
            copy_kernel<SB, DB, OP, H><<<grid, kCopyBlock, 0, s>>>(table, count, divisor, first, hints);
        }
    });
}

// Conversions and division for 4- and 2-byte elements; H: the 2-byte side is fp16.
// Division by a power of two (the AVG pre-divide at a power-of-two world size) runs as a
// multiply by the exact reciprocal: the same bits, without the division sequence.
template <bool H>
int32_t launch_arith(int ssz, int dsz, int32_t op, float divisor, const int64_t* table, int64_t count,
                     int64_t chunks, bool aligned, const int64_t* hints, hipStream_t s) {
    const float recip = op == HBT_COPY_OP_DIVIDE ? exact_reciprocal(divisor) : 0.0f;
    if (op == HBT_COPY_OP_DIVIDE && recip != 0.0f) {
        if (ssz == 4 && dsz == 4) return launch_copy<4, 4, kOpScale>(table, count, chunks, recip, aligned, hints, s);
        if (ssz == 2 && dsz == 2) return launch_copy<2, 2, kOpScale, H>(table, count, chunks, recip, aligned, hints, s);
        if (ssz == 4) return launch_copy<4, 2, kOpScale, H>(table, count, chunks, recip, aligned, hints, s);
        return launch_copy<2, 4, kOpScale, H>(table, count, chunks, recip, aligned, hints, s);
    }
    if (op == HBT_COPY_OP_DIVIDE) {
        if (ssz == 4 && dsz == 4) return launch_copy<4, 4, HBT_COPY_OP_DIVIDE>(table, count, chunks, divisor, aligned, hints, s);
        if (ssz == 2 && dsz == 2) return launch_copy<2, 2, HBT_COPY_OP_DIVIDE, H>(table, count, chunks, divisor, aligned, hints, s);
        if (ssz == 4) return launch_copy<4, 2, HBT_COPY_OP_DIVIDE, H>(table, count, chunks, divisor, aligned, hints, s);
        return launch_copy<2, 4, HBT_COPY_OP_DIVIDE, H>(table, count, chunks, divisor, aligned, hints, s);
    }
    // conversions (same-dtype copies are bit copies)
    if (ssz == 4) return launch_copy<4, 2, HBT_COPY_OP_COPY, H>(table, count, chunks, divisor, aligned, hints, s);
    return launch_copy<2, 4, HBT_COPY_OP_COPY, H>(table, count, chunks, divisor, aligned, hints, s);
}

}  // namespace
}  // namespace hbt

using namespace hbt;

extern "C" {

int64_t hbt_copy_chunk_elems(int32_t src_dtype, int32_t dst_dtype) {
    const int ssz = dtype_size(src_dtype);
    const int dsz = dtype_size(dst_dtype);
    if (ssz == 0 || dsz == 0) return -1;
    // 1 KB of source, 2 KB when widening (the convert kernels' chunks are the copy
    // kernels'); F64 -> F64: the chunk of the DIVIDE op (a same-dtype COPY moves F32 dword
    // pairs).
    return int64_t(kCopyBlock) * 16 / ssz * (ssz < dsz ? 2 : 1);
}

int32_t hbt_copy_intervals(const int64_t* table, int64_t count, int64_t total_chunks,
                           int32_t src_dtype, int32_t dst_dtype, int32_t op, float divisor,
                           int32_t flags, void* stream) {
    clear_error();
    if (count < 0 || total_chunks < 0 || (count > 0 && table == nullptr)) {
        set_error("hbt_copy_intervals: bad table/count/total_chunks");
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if ((flags & ~(HBT_COPY_ALIGNED | HBT_COPY_HINTS)) != 0) {
        set_error("hbt_copy_intervals: unknown flags 0x%x", static_cast<unsigned>(flags));
        return HBT_ERR_INVALID_ARGUMENT;
    }
    const bool aligned = (flags & HBT_COPY_ALIGNED) != 0;
    if (count == 0 || total_chunks == 0) return HBT_OK;
    // The hints follow the count records of 4 int64 each.
    const int64_t* hints = (flags & HBT_COPY_HINTS) != 0 ? table + 4 * count : nullptr;
    const int ssz = dtype_size(src_dtype);
    const int dsz = dtype_size(dst_dtype);
    if (ssz == 0 || dsz == 0 || (op != HBT_COPY_OP_COPY && op != HBT_COPY_OP_DIVIDE)) {
        set_error("hbt_copy_intervals: bad dtype pair (%d, %d) or op %d", src_dtype, dst_dtype, op);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    hipStream_t s = as_stream(stream);
    if (op == HBT_COPY_OP_DIVIDE && src_dtype == HBT_DTYPE_F64 && dst_dtype == HBT_DTYPE_F64) {
        const float recip = exact_reciprocal(divisor);
        if (recip != 0.0f)
            return launch_convert<kOpScale>(src_dtype, dst_dtype, table, count, total_chunks, recip, aligned, hints, s);
        return launch_convert<HBT_COPY_OP_DIVIDE>(src_dtype, dst_dtype, table, count, total_chunks, divisor, aligned,
                                                  hints, s);
    }
    if (op == HBT_COPY_OP_COPY && src_dtype == dst_dtype) {
        // Bit copy; fp64 moves as pairs of dwords (the host doubles its numels).
        if (ssz == 2) return launch_copy<2, 2, HBT_COPY_OP_COPY>(table, count, total_chunks, divisor, aligned, hints, s);
        if (ssz == 4) return launch_copy<4, 4, HBT_COPY_OP_COPY>(table, count, total_chunks, divisor, aligned, hints, s);
        set_error("hbt_copy_intervals: 8-byte elements must be passed as dword pairs (F32)");
        return HBT_ERR_UNSUPPORTED;
    }
    const bool wide = ssz == 8 || dsz == 8;
    const bool mixed_16 = (src_dtype == HBT_DTYPE_BF16 && dst_dtype == HBT_DTYPE_F16) ||
                          (src_dtype == HBT_DTYPE_F16 && dst_dtype == HBT_DTYPE_BF16);
    if (wide || mixed_16) {
        if (op != HBT_COPY_OP_COPY) {
            set_error("hbt_copy_intervals: division moves data within one dtype (F64, F32, BF16 or F16) or "
                      "between F32 and a 2-byte dtype (got %d -> %d)", src_dtype, dst_dtype);
            return HBT_ERR_UNSUPPORTED;
        }
        return launch_convert<HBT_COPY_OP_COPY>(src_dtype, dst_dtype, table, count, total_chunks, 1.0, aligned,
                                                hints, s);
    }
    if (src_dtype == HBT_DTYPE_F16 || dst_dtype == HBT_DTYPE_F16) {
        return launch_arith<true>(ssz, dsz, op, divisor, table, count, total_chunks, aligned, hints, s);
    }
    return launch_arith<false>(ssz, dsz, op, divisor, table, count, total_chunks, aligned, hints, s);
}

}  // extern "C"
