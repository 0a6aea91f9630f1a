// Interval gather-copy and the FSDP gradient local share (gfx950).
//
// One launch moves any number of [src, src + n) -> [dst, dst + n) intervals.  Each
// interval is cut into chunks of 512 elements; one workgroup owns one chunk
// and finds its interval by binary search over the records' first_chunk column.  Inside
// a chunk each lane moves units of 16 / max(source, destination element bytes)
// elements, consecutive lanes taking consecutive units, so every load and store
// instruction of a wave covers one contiguous span.  The destination is written with
// aligned stores; the source is read with aligned loads of the unit's width and
// shifted into place with v_alignbyte, so intervals at any element offset stream at
// full width.  A load never touches an aligned block that holds no byte of the source
// interval.
#include "hbt_common.hpp"

namespace hbt {
namespace {

// One wavefront per workgroup: a workgroup moves a 512-element chunk and retires.
// Measured on MI355X (Llama-3-8B bf16 reshard, 32 GB moved), this shape sustains
// 6.3 TB/s against 5.0 TB/s for 256-thread workgroups walking 64K-element chunks.
// Halving the chunk of 4-byte data (one unit per lane) measured slower in the
// product (6.6 -> 5.2 TB/s for bf16 -> fp32 packs): each workgroup's interval
// search is then paid twice per byte.
#ifndef HBT_COPY_BLOCK
#define HBT_COPY_BLOCK 64
#endif
#ifndef HBT_COPY_NT
#define HBT_COPY_NT 1
#endif
constexpr int kCopyBlock = HBT_COPY_BLOCK;
constexpr bool kCopyNT = HBT_COPY_NT != 0;

// Aligned vector load/store of NW dwords (NW = 2 or 4), non-temporal when kCopyNT:
// every byte is moved exactly once.
template <int NW>
struct Vec {
    typedef uint32_t type __attribute__((ext_vector_type(NW)));
};
typedef Vec<4>::type u32x4v;
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int NW>
__device__ __forceinline__ typename Vec<NW>::type ldv(const void* p) {
    typedef typename Vec<NW>::type V;
    if constexpr (kCopyNT) return __builtin_nontemporal_load(reinterpret_cast<const V*>(p));
    return *reinterpret_cast<const V*>(p);
}
template <int NW>
__device__ __forceinline__ void stv(void* p, typename Vec<NW>::type x) {
    typedef typename Vec<NW>::type V;
    if constexpr (kCopyNT) {
        __builtin_nontemporal_store(x, reinterpret_cast<V*>(p));
    } else {
        *reinterpret_cast<V*>(p) = x;
    }
}

// Loads NW dwords (NW = 2 or 4: one 8- or 16-byte block) starting at byte address
// `s`, where `k` = s mod 4*NW (uniform across the wave).  For k != 0 one extra aligned
// block is read; it holds source bytes s + 4*NW - 1 and earlier ones only up to the
// block boundary, so it lies inside the source's page.
template <int NW>
__device__ __forceinline__ void load_shifted(const uint8_t* s, uint32_t k, uint32_t (&out)[NW]) {
    static_assert(NW == 2 || NW == 4, "units are 8 or 16 bytes");
    const uint8_t* a = s - k;
    const typename Vec<NW>::type x = ldv<NW>(a);
    if (k == 0) {
#pragma unroll
        for (int i = 0; i < NW; ++i) out[i] = x[i];
        return;
    }
    const typename Vec<NW>::type y = ldv<NW>(a + 4 * NW);
    uint32_t w[2 * NW];
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        w[i] = x[i];
        w[NW + i] = y[i];
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

// Element semantics.  SB/DB are source/destination element bytes.  Same-size COPY is
// a bit copy; 4->2 narrows fp32 to bf16, 2->4 widens bf16 to fp32; DIVIDE goes through
// fp32 (true division) and rounds to the destination type.
template <int SB>
__device__ __forceinline__ float elem_to_f32(uint32_t bits) {
    if constexpr (SB == 4) return __uint_as_float(bits);
    return bf16_to_f32(bits);
}
template <int DB>
__device__ __forceinline__ uint32_t f32_to_elem(float x) {
    if constexpr (DB == 4) return __float_as_uint(x);
    return f32_to_bf16(x);
}
template <int SB, int DB, int OP>
__device__ __forceinline__ uint32_t convert(uint32_t bits, float divisor) {
    if constexpr (SB == DB && OP == HBT_COPY_OP_COPY) return bits;
    float x = elem_to_f32<SB>(bits);
    if constexpr (OP == HBT_COPY_OP_DIVIDE) x = x / divisor;
    return f32_to_elem<DB>(x);
}

template <int EB>
__device__ __forceinline__ uint32_t load_elem(const uint8_t* p) {
    if constexpr (EB == 4) return *reinterpret_cast<const uint32_t*>(p);
    return *reinterpret_cast<const uint16_t*>(p);
}
template <int EB>
__device__ __forceinline__ void store_elem(uint8_t* p, uint32_t bits) {
    if constexpr (EB == 4) {
        *reinterpret_cast<uint32_t*>(p) = bits;
    } else {
        *reinterpret_cast<uint16_t*>(p) = static_cast<uint16_t>(bits);
    }
}

// Elements per lane unit: one 16-byte access on the wider side of the copy.
template <int SB, int DB>
constexpr int unit_elems() { return 16 / (SB > DB ? SB : DB); }
// Elements per chunk (per workgroup), the same for every dtype pair.
template <int SB, int DB>
constexpr int64_t chunk_elems() { return 512; }

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
__device__ __forceinline__ void pack_unit_store(uint8_t* d, const uint32_t (&e)[U]) {
    constexpr int NW = U * DB / 4;
    typename Vec<NW>::type x;
    if constexpr (DB == 4) {
#pragma unroll
        for (int i = 0; i < U; ++i) x[i] = e[i];
    } else {
#pragma unroll
        for (int i = 0; i < U / 2; ++i) x[i] = e[2 * i] | (e[2 * i + 1] << 16);
    }
    stv<NW>(d, x);
}

template <int SB, int DB, int OP>
__global__ __launch_bounds__(kCopyBlock) void copy_kernel(const int64_t* __restrict__ table,
                                                          int64_t count, float divisor) {
    const int64_t chunk = static_cast<int64_t>(blockIdx.x);
    // Last record whose first_chunk <= chunk (records with no chunks are skipped by
    // the host, so this is the owning record).
    int64_t lo = 0, hi = count - 1;
    while (lo < hi) {
        const int64_t mid = (lo + hi + 1) >> 1;
        if (table[4 * mid + 3] <= chunk) {
            lo = mid;
        } else {
            hi = mid - 1;
        }
    }
    const int64_t* rec = table + 4 * lo;
    const uint8_t* src = reinterpret_cast<const uint8_t*>(rec[0]);
    uint8_t* dst = reinterpret_cast<uint8_t*>(rec[1]);
    const int64_t n = rec[2];
    constexpr int64_t kChunk = chunk_elems<SB, DB>();
    const int64_t e0 = (chunk - rec[3]) * kChunk;
    const int64_t len = (n - e0) < kChunk ? (n - e0) : kChunk;

    uint8_t* d = dst + e0 * DB;
    const uint8_t* s = src != nullptr ? src + e0 * SB : nullptr;

    // Head: elements until the destination is 16-byte aligned.
    int64_t head = static_cast<int64_t>(((16u - (reinterpret_cast<uintptr_t>(d) & 15u)) & 15u) / DB);
    if (head > len) head = len;
    constexpr int U = unit_elems<SB, DB>();
    const int64_t units = (len - head) / U;
    const int64_t tail_begin = head + units * U;

    if (threadIdx.x < head) {
        const int64_t e = threadIdx.x;
        const uint32_t bits = s != nullptr ? convert<SB, DB, OP>(load_elem<SB>(s + e * SB), divisor) : 0u;
        store_elem<DB>(d + e * DB, bits);
    }
    if (threadIdx.x < len - tail_begin) {
        const int64_t e = tail_begin + threadIdx.x;
        const uint32_t bits = s != nullptr ? convert<SB, DB, OP>(load_elem<SB>(s + e * SB), divisor) : 0u;
        store_elem<DB>(d + e * DB, bits);
    }

    uint8_t* dbody = d + head * DB;
    if (s == nullptr) {
        for (int64_t u = threadIdx.x; u < units; u += kCopyBlock) {
            uint32_t zero[U];
#pragma unroll
            for (int i = 0; i < U; ++i) zero[i] = 0u;
            pack_unit_store<DB, U>(dbody + u * U * DB, zero);
        }
        return;
    }
    const uint8_t* sbody = s + head * SB;
    constexpr int kSrcWords = U * SB / 4;
    const uint32_t k = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(sbody) & (4u * kSrcWords - 1u));
    for (int64_t u = threadIdx.x; u < units; u += kCopyBlock) {
        uint32_t words[kSrcWords];
        load_shifted<kSrcWords>(sbody + u * U * SB, k, words);
        uint32_t e[U];
        unpack_unit<SB, U>(words, e);
#pragma unroll
        for (int i = 0; i < U; ++i) e[i] = convert<SB, DB, OP>(e[i], divisor);
        pack_unit_store<DB, U>(dbody + u * U * DB, e);
    }
}

// ---- FSDP gradient local share -------------------------------------------------------
struct RankTable {
    const uint8_t* g[HBT_MAX_LOCAL_RANKS];
};

// One wavefront per workgroup and 256 shard elements per workgroup: each lane owns one
// 4-element group (fp32 input: one 16-byte load per rank; bf16 input: one 8-byte
// load), adds the G ranks' quotients in rank order and stores 16 bytes.  Measured on
// MI355X (8 bf16 ranks -> fp32): 6.0 TB/s, against 5.7 TB/s with two groups per lane.
constexpr int kShareBlock = 64;
constexpr int kShareGroups = 1;
constexpr int64_t kShareTile = int64_t(kShareBlock) * 4 * kShareGroups;

template <int SB>
__device__ __forceinline__ f32x4 load_quad(const uint8_t* p) {
    if constexpr (SB == 4) {
        const u32x4v w = ldv<4>(p);
        return f32x4{__uint_as_float(w.x), __uint_as_float(w.y), __uint_as_float(w.z), __uint_as_float(w.w)};
    } else {
        const typename Vec<2>::type w = ldv<2>(p);
        return f32x4{bf16_to_f32(w.x & 0xFFFFu), bf16_to_f32(w.x >> 16), bf16_to_f32(w.y & 0xFFFFu),
                     bf16_to_f32(w.y >> 16)};
    }
}

template <int SB>
__global__ __launch_bounds__(kShareBlock) void local_share_kernel(RankTable ranks, int32_t group_size,
                                                                  int64_t offset, int64_t shard_numel,
                                                                  int64_t valid_numel, float divisor,
                                                                  int32_t vec_ok,
                                                                  float* __restrict__ out) {
    const int64_t base = int64_t(blockIdx.x) * kShareTile;
    if (vec_ok && base + kShareTile <= valid_numel) {
#pragma unroll
        for (int u = 0; u < kShareGroups; ++u) {
            const int64_t e = base + (int64_t(u) * kShareBlock + threadIdx.x) * 4;
            f32x4 acc = load_quad<SB>(ranks.g[0] + (offset + e) * SB) / divisor;
            for (int32_t q = 1; q < group_size; ++q) {
                acc = acc + load_quad<SB>(ranks.g[q] + (offset + e) * SB) / divisor;
            }
            stv<4>(out + e, u32x4v{__float_as_uint(acc.x), __float_as_uint(acc.y),
                                     __float_as_uint(acc.z), __float_as_uint(acc.w)});
        }
        return;
    }
    if (vec_ok && base >= valid_numel && base + kShareTile <= shard_numel) {
#pragma unroll
        for (int u = 0; u < kShareGroups; ++u) {
            const int64_t e = base + (int64_t(u) * kShareBlock + threadIdx.x) * 4;
            stv<4>(out + e, u32x4v{0u, 0u, 0u, 0u});
        }
        return;
    }
    const int64_t end = base + kShareTile < shard_numel ? base + kShareTile : shard_numel;
    for (int64_t i = base + threadIdx.x; i < end; i += kShareBlock) {
        float acc = 0.0f;
        if (i < valid_numel) {
            acc = elem_to_f32<SB>(load_elem<SB>(ranks.g[0] + (offset + i) * SB)) / divisor;
            for (int32_t q = 1; q < group_size; ++q) {
                acc = acc + elem_to_f32<SB>(load_elem<SB>(ranks.g[q] + (offset + i) * SB)) / divisor;
            }
        }
        out[i] = acc;
    }
}

template <int SB, int DB, int OP>
void launch_copy(const int64_t* table, int64_t count, int64_t chunks, float divisor, hipStream_t s) {
    copy_kernel<SB, DB, OP><<<dim3(static_cast<unsigned>(chunks)), kCopyBlock, 0, s>>>(table, count, divisor);
}

}  // namespace
}  // namespace hbt

using namespace hbt;

extern "C" {

int64_t hbt_copy_chunk_elems(int32_t src_dtype, int32_t dst_dtype) {
    const int ssz = dtype_size(src_dtype);
    const int dsz = dtype_size(dst_dtype);
    if (ssz == 4 && dsz == 4) return chunk_elems<4, 4>();
    if (ssz == 2 && dsz == 2) return chunk_elems<2, 2>();
    if (ssz == 4 && dsz == 2) return chunk_elems<4, 2>();
    if (ssz == 2 && dsz == 4) return chunk_elems<2, 4>();
    return -1;  // 8-byte elements travel as F32 dword pairs
}

int32_t hbt_copy_intervals(const int64_t* table, int64_t count, int64_t total_chunks,
                           int32_t src_dtype, int32_t dst_dtype, int32_t op, float divisor,
                           void* stream) {
    clear_error();
    if (count < 0 || total_chunks < 0 || (count > 0 && table == nullptr)) {
        set_error("hbt_copy_intervals: bad table/count/total_chunks");
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if (count == 0 || total_chunks == 0) return HBT_OK;
    if (total_chunks > 0x7FFFFFFFLL) {
        set_error("hbt_copy_intervals: %lld chunks exceed the grid limit",
                  static_cast<long long>(total_chunks));
        return HBT_ERR_UNSUPPORTED;
    }
    const int ssz = dtype_size(src_dtype);
    const int dsz = dtype_size(dst_dtype);
    if (ssz == 0 || dsz == 0 || (op != HBT_COPY_OP_COPY && op != HBT_COPY_OP_DIVIDE)) {
        set_error("hbt_copy_intervals: bad dtype pair (%d, %d) or op %d", src_dtype, dst_dtype, op);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    const bool arithmetic = src_dtype == HBT_DTYPE_F32 || src_dtype == HBT_DTYPE_BF16;
    const bool arithmetic_dst = dst_dtype == HBT_DTYPE_F32 || dst_dtype == HBT_DTYPE_BF16;
    hipStream_t s = as_stream(stream);
    if (op == HBT_COPY_OP_COPY && src_dtype == dst_dtype) {
        // Bit copy; fp64 moves as pairs of dwords (the host doubles its numels).
        if (ssz == 2) {
            launch_copy<2, 2, HBT_COPY_OP_COPY>(table, count, total_chunks, divisor, s);
        } else if (ssz == 4) {
            launch_copy<4, 4, HBT_COPY_OP_COPY>(table, count, total_chunks, divisor, s);
        } else {
            set_error("hbt_copy_intervals: 8-byte elements must be passed as dword pairs (F32)");
            return HBT_ERR_UNSUPPORTED;
        }
        return check_launch("hbt_copy_intervals");
    }
    if (!arithmetic || !arithmetic_dst) {
        set_error("hbt_copy_intervals: conversions and division support F32 and BF16 only");
        return HBT_ERR_UNSUPPORTED;
    }
    const bool div = op == HBT_COPY_OP_DIVIDE;
    if (ssz == 4 && dsz == 4) {
        launch_copy<4, 4, HBT_COPY_OP_DIVIDE>(table, count, total_chunks, divisor, s);
    } else if (ssz == 2 && dsz == 2) {
        launch_copy<2, 2, HBT_COPY_OP_DIVIDE>(table, count, total_chunks, divisor, s);
    } else if (ssz == 4 && dsz == 2) {
        if (div) {
            launch_copy<4, 2, HBT_COPY_OP_DIVIDE>(table, count, total_chunks, divisor, s);
        } else {
            launch_copy<4, 2, HBT_COPY_OP_COPY>(table, count, total_chunks, divisor, s);
        }
    } else {
        if (div) {
            launch_copy<2, 4, HBT_COPY_OP_DIVIDE>(table, count, total_chunks, divisor, s);
        } else {
            launch_copy<2, 4, HBT_COPY_OP_COPY>(table, count, total_chunks, divisor, s);
        }
    }
    return check_launch("hbt_copy_intervals");
}

int32_t hbt_grad_local_share(const void* const* rank_grads, int32_t group_size, int32_t rank,
                             int64_t shard_numel, int64_t valid_numel, int32_t in_dtype,
                             float divisor, float* out, void* stream) {
    clear_error();
    if (rank_grads == nullptr || out == nullptr || group_size < 1 ||
        group_size > HBT_MAX_LOCAL_RANKS || rank < 0 || rank >= group_size || shard_numel < 0 ||
        valid_numel < 0 || valid_numel > shard_numel) {
        set_error("hbt_grad_local_share: bad arguments (group_size=%d rank=%d shard=%lld valid=%lld)",
                  group_size, rank, static_cast<long long>(shard_numel),
                  static_cast<long long>(valid_numel));
        return HBT_ERR_INVALID_ARGUMENT;
    }
    if (in_dtype != HBT_DTYPE_F32 && in_dtype != HBT_DTYPE_BF16) {
        set_error("hbt_grad_local_share: input dtype %d is not F32 or BF16", in_dtype);
        return HBT_ERR_INVALID_ARGUMENT;
    }
    RankTable ranks{};
    for (int q = 0; q < group_size; ++q) {
        if (rank_grads[q] == nullptr && valid_numel > 0) {
            set_error("hbt_grad_local_share: rank %d gradient pointer is null", q);
            return HBT_ERR_INVALID_ARGUMENT;
        }
        ranks.g[q] = static_cast<const uint8_t*>(rank_grads[q]);
    }
    if (shard_numel == 0) return HBT_OK;
    const int64_t offset = int64_t(rank) * shard_numel;
    const int64_t tiles = (shard_numel + kShareTile - 1) / kShareTile;
    if (tiles > 0x7FFFFFFFLL) {
        set_error("hbt_grad_local_share: %lld tiles exceed the grid limit", static_cast<long long>(tiles));
        return HBT_ERR_UNSUPPORTED;
    }
    // Vector path: every rank's slice and the output start on a 16-byte (fp32 input) or
    // 8-byte (bf16 input) boundary.
    const int elem = in_dtype == HBT_DTYPE_F32 ? 4 : 2;
    int32_t vec_ok = (reinterpret_cast<uintptr_t>(out) & 15u) == 0;
    for (int q = 0; q < group_size && vec_ok; ++q) {
        const uintptr_t a = reinterpret_cast<uintptr_t>(ranks.g[q]) + static_cast<uintptr_t>(offset * elem);
        vec_ok = (a & static_cast<uintptr_t>(4 * elem - 1)) == 0;
    }
    hipStream_t s = as_stream(stream);
    if (in_dtype == HBT_DTYPE_F32) {
        local_share_kernel<4><<<dim3(static_cast<unsigned>(tiles)), kShareBlock, 0, s>>>(
            ranks, group_size, offset, shard_numel, valid_numel, divisor, vec_ok, out);
    } else {
        local_share_kernel<2><<<dim3(static_cast<unsigned>(tiles)), kShareBlock, 0, s>>>(
            ranks, group_size, offset, shard_numel, valid_numel, divisor, vec_ok, out);
    }
    return check_launch("hbt_grad_local_share");
}

}  // extern "C"
