// Interval gather-copy and the FSDP gradient local share (gfx950).
//
// One launch moves any number of [src, src + n) -> [dst, dst + n) intervals.  Each
// interval is cut into chunks of kCopyChunk elements; one workgroup owns one chunk
// and finds its interval by binary search over the records' first_chunk column.  Inside
// a chunk the destination is written with aligned 16-byte stores; the source is read
// with aligned 16-byte loads and shifted into place with v_alignbyte, so intervals at
// any element offset stream at full width.  A load never touches a 16-byte block that
// holds no byte of the source interval.
#include "hbt_common.hpp"

namespace hbt {
namespace {

// One wavefront per workgroup and one 8-element unit per lane: a workgroup moves a
// 512-element chunk and retires.  Measured on MI355X (Llama-3-8B bf16 reshard, 32 GB
// moved), this shape sustains 6.3 TB/s against 5.0 TB/s for 256-thread workgroups
// walking 64K-element chunks.
#ifndef HBT_COPY_BLOCK
#define HBT_COPY_BLOCK 64
#endif
#ifndef HBT_COPY_CHUNK
#define HBT_COPY_CHUNK 512
#endif
#ifndef HBT_COPY_UNROLL
#define HBT_COPY_UNROLL 1
#endif
#ifndef HBT_COPY_NT
#define HBT_COPY_NT 1
#endif
constexpr int kCopyBlock = HBT_COPY_BLOCK;
constexpr int64_t kCopyChunk = HBT_COPY_CHUNK;  // elements per block
constexpr int kCopyUnroll = HBT_COPY_UNROLL;    // 8-element units per thread per iteration
constexpr bool kCopyNT = HBT_COPY_NT != 0;

typedef uint32_t u32x4_nt __attribute__((ext_vector_type(4)));
// 16-byte load/store, non-temporal when kCopyNT: every byte is moved exactly once.
__device__ __forceinline__ u32x4_nt ld16(const void* p) {
    if constexpr (kCopyNT) return __builtin_nontemporal_load(reinterpret_cast<const u32x4_nt*>(p));
    return *reinterpret_cast<const u32x4_nt*>(p);
}
__device__ __forceinline__ void st16(void* p, u32x4_nt x) {
    if constexpr (kCopyNT) {
        __builtin_nontemporal_store(x, reinterpret_cast<u32x4_nt*>(p));
    } else {
        *reinterpret_cast<u32x4_nt*>(p) = x;
    }
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Loads NW dwords starting at byte address `s`, where `k` = s & 15 (uniform across the
// wave).  For k != 0 one extra aligned block is read; it holds source bytes s+NW*4-1
// and earlier ones only up to the block boundary, so it lies inside the source's page.
template <int NW>
__device__ __forceinline__ void load_shifted(const uint8_t* s, uint32_t k, uint32_t (&out)[NW]) {
    static_assert(NW == 4 || NW == 8, "units are 16 or 32 bytes");
    constexpr int kBlocks = NW / 4;
    const uint8_t* a = s - k;
    if (k == 0) {
#pragma unroll
        for (int b = 0; b < kBlocks; ++b) {
            const u32x4 x = ld16(a + 16 * b);
            out[4 * b + 0] = x.x;
            out[4 * b + 1] = x.y;
            out[4 * b + 2] = x.z;
            out[4 * b + 3] = x.w;
        }
        return;
    }
    uint32_t w[NW + 4];
#pragma unroll
    for (int b = 0; b <= kBlocks; ++b) {
        const u32x4 x = ld16(a + 16 * b);
        w[4 * b + 0] = x.x;
        w[4 * b + 1] = x.y;
        w[4 * b + 2] = x.z;
        w[4 * b + 3] = x.w;
    }
    const uint32_t r = k & 3u;
    switch (k >> 2) {
        case 0:
#pragma unroll
            for (int i = 0; i < NW; ++i) out[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], r);
            break;
        case 1:
#pragma unroll
            for (int i = 0; i < NW; ++i) out[i] = __builtin_amdgcn_alignbyte(w[i + 2], w[i + 1], r);
            break;
        case 2:
#pragma unroll
            for (int i = 0; i < NW; ++i) out[i] = __builtin_amdgcn_alignbyte(w[i + 3], w[i + 2], r);
            break;
        default:
#pragma unroll
            for (int i = 0; i < NW; ++i) out[i] = __builtin_amdgcn_alignbyte(w[i + 4], w[i + 3], r);
            break;
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

// Unpack the 8 elements held in `words` (SB bytes each) into element bit patterns.
template <int SB>
__device__ __forceinline__ void unpack8(const uint32_t (&words)[2 * SB], uint32_t (&e)[8]) {
    if constexpr (SB == 4) {
#pragma unroll
        for (int i = 0; i < 8; ++i) e[i] = words[i];
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            e[2 * i] = words[i] & 0xFFFFu;
            e[2 * i + 1] = words[i] >> 16;
        }
    }
}
template <int DB>
__device__ __forceinline__ void pack8_store(uint8_t* d, const uint32_t (&e)[8]) {
    if constexpr (DB == 4) {
        st16(d, u32x4{e[0], e[1], e[2], e[3]});
        st16(d + 16, u32x4{e[4], e[5], e[6], e[7]});
    } else {
        st16(d, u32x4{e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16), e[6] | (e[7] << 16)});
    }
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
    const int64_t e0 = (chunk - rec[3]) * kCopyChunk;
    const int64_t len = (n - e0) < kCopyChunk ? (n - e0) : kCopyChunk;

    uint8_t* d = dst + e0 * DB;
    const uint8_t* s = src != nullptr ? src + e0 * SB : nullptr;

    // Head: elements until the destination is 16-byte aligned.
    int64_t head = static_cast<int64_t>(((16u - (reinterpret_cast<uintptr_t>(d) & 15u)) & 15u) / DB);
    if (head > len) head = len;
    const int64_t units = (len - head) / 8;
    const int64_t tail_begin = head + units * 8;

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
            const uint32_t zero[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            pack8_store<DB>(dbody + u * 8 * DB, zero);
        }
        return;
    }
    const uint8_t* sbody = s + head * SB;
    const uint32_t k = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(sbody) & 15u);
    int64_t u = threadIdx.x;
    for (; u + int64_t(kCopyUnroll - 1) * kCopyBlock < units; u += int64_t(kCopyUnroll) * kCopyBlock) {
        uint32_t words[kCopyUnroll][2 * SB];
#pragma unroll
        for (int j = 0; j < kCopyUnroll; ++j) {
            load_shifted<2 * SB>(sbody + (u + int64_t(j) * kCopyBlock) * 8 * SB, k, words[j]);
        }
#pragma unroll
        for (int j = 0; j < kCopyUnroll; ++j) {
            uint32_t e[8];
            unpack8<SB>(words[j], e);
#pragma unroll
            for (int i = 0; i < 8; ++i) e[i] = convert<SB, DB, OP>(e[i], divisor);
            pack8_store<DB>(dbody + (u + int64_t(j) * kCopyBlock) * 8 * DB, e);
        }
    }
    for (; u < units; u += kCopyBlock) {
        uint32_t words[2 * SB];
        load_shifted<2 * SB>(sbody + u * 8 * SB, k, words);
        uint32_t e[8];
        unpack8<SB>(words, e);
#pragma unroll
        for (int i = 0; i < 8; ++i) e[i] = convert<SB, DB, OP>(e[i], divisor);
        pack8_store<DB>(dbody + u * 8 * DB, e);
    }
}

// ---- FSDP gradient local share -------------------------------------------------------
struct RankTable {
    const uint8_t* g[HBT_MAX_LOCAL_RANKS];
};

template <int SB>
__global__ __launch_bounds__(256) void local_share_kernel(RankTable ranks, int32_t group_size,
                                                          int64_t offset, int64_t shard_numel,
                                                          int64_t valid_numel, float divisor,
                                                          float* __restrict__ out) {
    const int64_t stride = int64_t(gridDim.x) * 256;
    for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < shard_numel; i += stride) {
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

int64_t hbt_copy_chunk_elems(void) { return kCopyChunk; }

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
    int64_t blocks = (shard_numel + 255) / 256;
    const int64_t cap = int64_t(device_cu_count()) * 16;
    if (blocks > cap) blocks = cap;
    const int64_t offset = int64_t(rank) * shard_numel;
    hipStream_t s = as_stream(stream);
    if (in_dtype == HBT_DTYPE_F32) {
        local_share_kernel<4><<<dim3(static_cast<unsigned>(blocks)), 256, 0, s>>>(
            ranks, group_size, offset, shard_numel, valid_numel, divisor, out);
    } else {
        local_share_kernel<2><<<dim3(static_cast<unsigned>(blocks)), 256, 0, s>>>(
            ranks, group_size, offset, shard_numel, valid_numel, divisor, out);
    }
    return check_launch("hbt_grad_local_share");
}

}  // extern "C"
