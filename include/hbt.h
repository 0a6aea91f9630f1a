/*
 * hbt.h - C ABI of the MI355X (gfx950) data-parallel hot-path library, libhbt.so.
 *
 * Every entry point takes plain device pointers, element counts, host scalars and a
 * hipStream_t passed as void*.  No torch types cross this boundary.  All work is
 * stream-ordered and asynchronous: an entry point returns once its kernels are
 * enqueued.  The return value is HBT_OK (0) or a negative status; hbt_last_error()
 * then holds a message for the calling thread.
 *
 * The reference (sdivyanshu90/build-your-own-hybrid-distributed-training, pure
 * Python) has no FFI of its own.  Each entry point below names the reference
 * function(s) whose torch op sequence it replaces, by file:line relative to the
 * reference's src/hybrid_training/ directory, or relative to the installed torch
 * package for the AdamW arithmetic the reference delegates to.
 */
#ifndef HBT_H
#define HBT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------------- */
#define HBT_OK 0
#define HBT_ERR_INVALID_ARGUMENT (-1) /* null pointer, negative size, bad dtype/op  */
#define HBT_ERR_UNSUPPORTED (-2)      /* legal request libhbt does not handle       */
#define HBT_ERR_HIP (-3)              /* a HIP runtime call or kernel launch failed */

/* ---- element types ----------------------------------------------------------- */
#define HBT_DTYPE_F32 0
#define HBT_DTYPE_BF16 1
#define HBT_DTYPE_F16 2
#define HBT_DTYPE_F64 3 /* float64: the _f64 optimizer entry points, norms, copies, conversions,
                           local-share reduce and master dtype, accumulate dtype */

/* ---- per-call limits ---------------------------------------------------------- */
#define HBT_MAX_TENSORS_PER_LAUNCH 16 /* AdamW / norm tables; the host splits larger lists */

/* Message describing the last failed call on this thread ("" if none). */
const char* hbt_last_error(void);

/* ABI version of the loaded library; the Python loader refuses a mismatch. */
int32_t hbt_abi_version(void);

/* Number of HBT_* entry points exported (used by the loader's symbol check). */
int32_t hbt_symbol_count(void);

/* How the library splits a grid of `blocks` workgroups of `threads` lanes into launches:
 * a HIP grid dimension holds at most 2^32 - 1 work-items, so each launch takes at most
 * floor((2^32 - 1) / threads) workgroups.  Writes the first block and the block count of
 * up to `capacity` slices to first[] / count[] (either may be NULL) and returns the number
 * of slices (0 for blocks <= 0, -1 for threads <= 0).  Every kernel launch in the library
 * goes through this split, so no request is refused for its size alone. */
int64_t hbt_grid_slices(int64_t blocks, int32_t threads, int64_t* first, int64_t* count, int64_t capacity);

/* ------------------------------------------------------------------------------
 * Fused gradient-clip + AdamW step over up to HBT_MAX_TENSORS_PER_LAUNCH tensors.
 *
 * Replaces: ShardedOptimizer.step (optim/sharded_optimizer.py:340-355) ->
 *   torch.optim.AdamW built at optim/sharded_optimizer.py:111-120 ->
 *   torch/optim/adam.py:396-547 (_single_tensor_adam, decoupled weight decay),
 *   preceded by the clip multiply of ShardedOptimizer.clip_grad_norm
 *   (optim/sharded_optimizer.py:333-337) and, for loss-scaled gradients, the
 *   unscale multiply of GradScaler.unscale_ (optim/grad_scaler.py:181-186).
 *
 * Dtypes (param_dtype for params, exp_avgs and exp_avg_sqs; grad_dtype for grads):
 * (F32, F32), (F32, BF16), (BF16, BF16) or (F16, F16).  Per element, in this order,
 * every operation computed in fp32 and rounded once; R_G rounds to the gradient's
 * dtype and R_P to the parameter's (both the identity for fp32):
 *   g  = R_G(g_in * unscale)       (skipped when unscale == 1)
 *   g  = R_G(g * (*grad_mul))      (grad_mul: device fp32 written by
 *                                   hbt_grad_norm_finalize, or NULL for 1)
 *   p  = R_P(p * decay)            (decay = fp32(1 - lr*weight_decay))
 *   m  = R_P(fma(w, g - m, m))     if |w| < 0.5, else R_P(fma(w - 1, g - m, g))
 *                                  (w = fp32(1 - beta1); lerp in its fused form)
 *   v  = R_P(v * beta2)
 *   v  = R_P(fma(one_minus_beta2 * g, g, v))
 *   d  = sqrt(v) / bias_correction2_sqrt + eps                      (fp32 parameters)
 *   d  = R_P(R_P(R_P(sqrt(v)) / bias_correction2_sqrt) + R_P(eps))  (2-byte parameters)
 *   p  = R_P(p + (neg_step_size * m) / d)
 * Each R_G is the gradient's in-place grad.mul_ of the reference, and each R_P one torch
 * CPU op on a tensor of the parameter dtype (torch rounds the scalar of add_(eps) to
 * that dtype).  sqrt and the divisions are correctly rounded.  The host computes the
 * scalars in double exactly as torch does and rounds them to fp32.
 *
 * flags: 0, or HBT_STEP_WRITE_GRAD to store the scaled gradient g back into grads[i]
 * (in its own dtype) whenever a multiply changed it, i.e. when unscale != 1 or
 * *grad_mul != 1.  That is the reference's in-place clip (and unscale) folded into the
 * update pass: one read and one write of g instead of a separate scaling pass.
 * Each tensor i has numels[i] elements; numels[i] may be 0.
 * ---------------------------------------------------------------------------- */
#define HBT_STEP_WRITE_GRAD 16
int32_t hbt_adamw_step(void* const* params, void* const* grads, void* const* exp_avgs,
                       void* const* exp_avg_sqs, const int64_t* numels, int32_t count,
                       int32_t param_dtype, int32_t grad_dtype, float unscale, const float* grad_mul,
                       float decay, float lerp_weight, float beta2, float one_minus_beta2,
                       float bias_correction2_sqrt, float eps, float neg_step_size, int32_t flags,
                       void* stream);

/* ------------------------------------------------------------------------------
 * Fused gradient-clip + SGD step over up to HBT_MAX_TENSORS_PER_LAUNCH tensors.
 *
 * Replaces: ShardedOptimizer.step (optim/sharded_optimizer.py:340-355) ->
 *   torch.optim.SGD built at optim/sharded_optimizer.py:121-126 ->
 *   torch/optim/sgd.py (_single_tensor_sgd), preceded by the clip and unscale
 *   multiplies as in hbt_adamw_step.
 * Dtypes as for hbt_adamw_step (momentum_buffers in param_dtype).  Per element, with
 * fma() a single rounding as torch's CPU `add(.., alpha=)`, R_G / R_P as above, and
 * a(x) = R_P(x): torch rounds every alpha to the parameter dtype first:
 *   g = R_G(R_G(g_in * unscale) * (*grad_mul))   (unscale skipped when 1; grad_mul NULL = 1)
 *   if HBT_SGD_WEIGHT_DECAY:  g = R_P(fma(p, a(weight_decay), g))
 *   if HBT_SGD_MOMENTUM:
 *       if HBT_SGD_FIRST_STEP: buf = g
 *       else:                  buf = R_P(fma(g, a(one_minus_dampening), R_P(buf * momentum)))
 *       g = HBT_SGD_NESTEROV ? R_P(fma(buf, a(momentum), g)) : buf
 *   p = R_P(fma(g, a(neg_lr), p))
 * momentum_buffers may be NULL without HBT_SGD_MOMENTUM.  Flags other than the four
 * below and HBT_STEP_WRITE_GRAD (as for hbt_adamw_step), or FIRST_STEP / NESTEROV
 * without MOMENTUM, are rejected.
 * ---------------------------------------------------------------------------- */
#define HBT_SGD_MOMENTUM 1
#define HBT_SGD_FIRST_STEP 2
#define HBT_SGD_NESTEROV 4
#define HBT_SGD_WEIGHT_DECAY 8
int32_t hbt_sgd_step(void* const* params, void* const* grads, void* const* momentum_buffers,
                     const int64_t* numels, int32_t count, int32_t param_dtype, int32_t grad_dtype,
                     float unscale, const float* grad_mul, float weight_decay, float momentum,
                     float one_minus_dampening, float neg_lr, int32_t flags, void* stream);

/* ------------------------------------------------------------------------------
 * Deterministic squared L2 norm, stage 1: per-block fp64 partial sums.
 *
 * Replaces: NormContribution.squared_norm (optim/sharded_optimizer.py:145-158)
 *   summed by distributed_gradient_norm (optim/sharded_optimizer.py:236-238).
 * Computes sum_i weights[i] * sum_j (double)(R_G(g_ij * unscale))^2 over up to
 * HBT_MAX_TENSORS_PER_LAUNCH gradient tensors (grad_dtype F32, BF16 or F16; R_G rounds
 * the unscaled value to that dtype, as the in-place unscale would have stored it; or F64
 * with unscale 1, each square one rounded double product), writing
 * hbt_norm_partials_count(numels, count, grad_dtype) doubles to partials: one per chunk
 * of consecutive elements of one tensor (32768 fp32, 65536 bf16/fp16, 16384 float64),
 * already multiplied by that tensor's weight.  The chunk -> partial map and every summation order depend only on the
 * numels, so the result is bitwise reproducible.  A non-finite element makes the
 * sum non-finite, which is the overflow signal of GradScaler._detect_non_finite
 * (optim/grad_scaler.py:189-200).
 * ---------------------------------------------------------------------------- */
int64_t hbt_norm_partials_count(const int64_t* numels, int32_t count, int32_t grad_dtype);
int32_t hbt_grad_sqnorm_partials(const void* const* grads, const int64_t* numels,
                                 const double* weights, int32_t count, int32_t grad_dtype,
                                 float unscale, double* partials, void* stream);

/* ------------------------------------------------------------------------------
 * Stage 2: fixed-order sum of `count` partials, sqrt, clip coefficient.
 *
 * Replaces: distributed_gradient_norm's clamp_min(0).sqrt()
 *   (optim/sharded_optimizer.py:241) and the clip-coefficient arithmetic of
 *   ShardedOptimizer.clip_grad_norm (optim/sharded_optimizer.py:331-337).
 * Writes sum_out[0] = the fp64 sum (if sum_out is non-NULL) and norm_out[0] =
 * sqrt(max(sum, 0)) (if norm_out is non-NULL).  The clip multiplier is
 * coef = max_norm / (norm + 1e-6) when max_norm > 0 and coef < 1, else 1: grad_mul_out
 * (if non-NULL) receives fp32(coef), the value torch multiplies fp32, bf16 and fp16
 * gradients by, and grad_mul64_out (if non-NULL) the double coef float64 gradients are
 * multiplied by.  If nonfinite_out is non-NULL it writes 1 when the sum is not finite,
 * else 0.  In a multi-rank job the stage-1 sum is what an fp64 all-reduce would combine
 * between the two stages.
 * ---------------------------------------------------------------------------- */
int32_t hbt_grad_norm_finalize(const double* partials, int64_t count, double max_norm,
                               double* sum_out, double* norm_out, float* grad_mul_out,
                               double* grad_mul64_out, int32_t* nonfinite_out, void* stream);

/* ------------------------------------------------------------------------------
 * Weighted squared norm and clip coefficient with no allocation and no workspace.
 *
 * This entry point has no counterpart in the reference.  It is for callers that
 * cannot allocate device memory: code under HIP graph capture, serving loops, or
 * harnesses that forbid hipMalloc.  It computes exactly what hbt_grad_sqnorm_partials
 * followed by hbt_grad_norm_finalize computes (same kernels, same partials layout,
 * same summation order, so the outputs are bitwise equal), but keeps the partials in
 * a static device array of HBT_NOALLOC_MAX_PARTIALS doubles (2 MiB per device, held
 * until the process ends) instead of a caller workspace.  It calls no hipMalloc,
 * hipFree or other allocating routine.  grad_dtype F32, BF16 or F16 (F64 returns
 * HBT_ERR_UNSUPPORTED).  The first call on a device looks up the array's device address;
 * make it outside graph capture.
 * Limit: hbt_norm_partials_count(numels, count, grad_dtype) must not exceed
 * HBT_NOALLOC_MAX_PARTIALS (8,589,934,592 fp32 or 17,179,869,184 bf16 elements per
 * call); a larger request returns HBT_ERR_UNSUPPORTED before any launch.
 * Every call on one device shares that device's array: calls that overlap in time on
 * one device (on different streams, or from different host threads) race.  Calls
 * ordered on one stream do not.  The outputs are as for hbt_grad_norm_finalize.
 * ---------------------------------------------------------------------------- */
#define HBT_NOALLOC_MAX_PARTIALS 262144
int32_t hbt_grad_norm_noalloc(const void* const* grads, const int64_t* numels, const double* weights,
                              int32_t count, int32_t grad_dtype, float unscale, double max_norm,
                              double* sum_out, double* norm_out, float* grad_mul_out,
                              int32_t* nonfinite_out, void* stream);

/* ------------------------------------------------------------------------------
 * Interval gather-copy: the one data-movement kernel behind flat-parameter
 * pack/pad/shard, unpack, DDP bucket pack with the AVG pre-divide, and
 * checkpoint interval resharding.
 *
 * Replaces:
 *   FlatParamHandle._build_shard     (parallel/fsdp.py:434-454)     pack + zero pad
 *   flatten_dense_tensors            (utils/tensors.py:199-260)     pack
 *   FlatParamHandle.full_tensors     (parallel/fsdp.py:912-925)     unpack copy
 *   FlatParamHandle.load_local_pieces(parallel/fsdp.py:862-910)     full -> shard slice
 *   _on_grad_ready pack + all_reduce AVG pre-divide
 *                                    (parallel/ddp.py:513, distributed/collectives.py:366-367)
 *   read_tensor_range                (checkpoint/reshard.py:200-305) interval copy
 *   FSDP destination fill            (checkpoint/reader.py:328-351, :423-443)
 *
 * `table` is a DEVICE array of `count` records of 4 int64 each:
 *   { src_address (0 => write zeros), dst_address, numel, first_chunk }
 * where first_chunk is the exclusive prefix sum over records of
 * ceil(numel / hbt_copy_chunk_elems(src_dtype, dst_dtype)), and total_chunks is the
 * sum.  A chunk is 1 KB of source: 128 elements of an 8-byte source, 256 of a 4-byte
 * one, 512 of a 2-byte one, except 2 KB when the destination is wider (1024 elements for
 * BF16/F16 -> F32 or F64, 512 for F32 -> F64), whose workgroups write more than they read;
 * hbt_copy_chunk_elems returns -1 for unknown dtypes.
 * A same-dtype F64 COPY travels as F32 dword pairs (the numels doubled); F64 -> F64 with
 * src_dtype = dst_dtype = F64 is the DIVIDE op's.  All records share src_dtype/dst_dtype and op:
 *   HBT_COPY_OP_COPY    dst = src               (same dtype: byte copy; F32->BF16
 *                                                rounds to nearest even, NaN -> 0x7FC0;
 *                                                F32->F16 rounds to nearest even, overflows
 *                                                to inf, keeps subnormals; BF16->F32 and
 *                                                F16->F32 widen exactly; an fp16 NaN keeps
 *                                                its sign and gets the quiet bit, with the
 *                                                payload kept (widening) or its top 10 bits
 *                                                kept (narrowing), as x86 F16C and torch's
 *                                                vectorised CPU conversions do)
 *                                               F64 -> F32/BF16/F16 and BF16 <-> F16 convert
 *                                                as torch's Tensor.to does: through the exact
 *                                                or nearest-even fp32 value, then to nearest
 *                                                even in the 2-byte dtype; F32/BF16/F16 -> F64
 *                                                widen exactly)
 *   HBT_COPY_OP_DIVIDE  dst = src / divisor     (true fp32 division, in fp32 for F32, BF16
 *                                                and F16 data, result rounded to dst_dtype;
 *                                                F64 -> F64 divides in double, correctly
 *                                                rounded, as div_ on a float64 tensor does;
 *                                                not for other F64 or BF16 <-> F16 pairs)
 * Source and destination ranges of one call must not overlap.  Addresses need no
 * particular alignment.
 *
 * flags: a combination of HBT_COPY_ALIGNED and HBT_COPY_HINTS.
 * HBT_COPY_HINTS: the table continues after the `count` records with
 * ceil(total_chunks / 256) int64 hints, hint j being the index of the record that owns
 * chunk 256 * j (the last record whose first_chunk <= 256 * j).  A workgroup then finds
 * its record by stepping forward from the hint instead of bisecting the table: on the
 * 148-record GPT-2-small bucket pack that search sits in front of every 1 KB copy.
 * HBT_COPY_ALIGNED when the caller certifies that every record's
 * dst_address is a multiple of 16 and every nonzero src_address a multiple of the
 * source width of one 16-byte destination-or-source unit, 16 * S / max(S, D) bytes for
 * S- and D-byte elements (16 for F32 -> F32, 8 for BF16 or F16 -> F32, 16 for the others).
 * Aligned plans run a kernel without the head and shifted-load paths (measured 6.6
 * against 5.7 TB/s on a 298-record fp32 unpack).  The results are the same bits
 * either way.
 * ---------------------------------------------------------------------------- */
#define HBT_COPY_OP_COPY 0
#define HBT_COPY_OP_DIVIDE 1
#define HBT_COPY_ALIGNED 1
#define HBT_COPY_HINTS 2
int64_t hbt_copy_chunk_elems(int32_t src_dtype, int32_t dst_dtype);
int32_t hbt_copy_intervals(const int64_t* table, int64_t count, int64_t total_chunks,
                           int32_t src_dtype, int32_t dst_dtype, int32_t op, float divisor,
                           int32_t flags, void* stream);

/* ------------------------------------------------------------------------------
 * FSDP gradient local share on one device.
 *
 * Replaces: FlatParamHandle.reduce_scatter_gradient (parallel/fsdp.py:704-769) with
 *   reduce_scatter_tensor AVG (distributed/collectives.py:588-595) and
 *   _zero_padding_region (parallel/fsdp.py:771-781).
 * `rank_grads` is a HOST array of `group_size` (at most HBT_MAX_LOCAL_RANKS) device
 * addresses, each the padded full gradient (group_size * shard_numel elements,
 * in_dtype F32, BF16 or F16) of one rank, all resident on this device.  Only elements
 * [rank*shard_numel, (rank+1)*shard_numel) of each are read, so a caller holding just
 * those slices (as the no_sync accumulator does) passes them with rank 0.  Writes the
 * shard of `rank` in out_dtype (the master dtype: F32, BF16 or F16), reducing in
 * `reduce_dtype` (F32, BF16 or F16), with R rounding to it (round to nearest even; the
 * identity for F32):
 *   x_q    = R(rank_grads[q][rank*shard_numel + i])   (the cast; none if in_dtype ==
 *                                                      reduce_dtype)
 *   s      = R(...R(R(x_0 / divisor) + R(x_1 / divisor)) + ... + R(x_{G-1} / divisor))
 * in rank order, each quotient and sum computed in fp32 and rounded once, as torch's
 * ops in that dtype give (divisor = G for AVG, 1 for SUM); then out[i] = s cast to
 * out_dtype (round to nearest even; exact when it is as wide), and +0.0 for
 * i >= valid_numel (the padding tail).  With group_size == 1 this is the whole local
 * share of one rank: cast to the reduce dtype, AVG pre-divide, cast to the master
 * dtype, zero padding.
 * reduce_dtype F64 (which also admits in_dtype F64, the float64 no_sync accumulator)
 * computes in double instead: s = ((x_0 / divisor + x_1 / divisor) + ...), each x_q
 * widened exactly, each quotient and sum correctly rounded in double, and s narrows to
 * out_dtype as Tensor.to does (to fp32 rounding to nearest even, then to a 2-byte
 * out_dtype), as torch's float64 ops give.
 * ---------------------------------------------------------------------------- */
#define HBT_MAX_LOCAL_RANKS 64
int32_t hbt_grad_local_share(const void* const* rank_grads, int32_t group_size, int32_t rank,
                             int64_t shard_numel, int64_t valid_numel, int32_t in_dtype,
                             int32_t reduce_dtype, float divisor, int32_t out_dtype, void* out, void* stream);

/* ------------------------------------------------------------------------------
 * FSDP gradient local share fused with the squared-norm partials of its output.
 *
 * Replaces: the same reference lines as hbt_grad_local_share, followed by the
 *   NormContribution.squared_norm pass over the produced shard
 *   (optim/sharded_optimizer.py:145-158) that the next clip_grad_norm runs.
 * Writes `out` exactly as hbt_grad_local_share does, and to `partials` the unweighted
 * squared norms of out's two segments, [0, valid_numel) then [valid_numel,
 * shard_numel), chunk by chunk: ceil(valid_numel / C) + ceil((shard_numel -
 * valid_numel) / C) doubles, one per C-element chunk from each segment's start (C =
 * 32768 for an F32 out_dtype, 65536 for a 2-byte one), in the layout
 * hbt_grad_sqnorm_partials uses for those segments (out_dtype, weight 1, unscale 1), so
 * a caller can stand them in for that pass.  Each is summed in a
 * fixed order (per 256-element tile, then per chunk), so it is reproducible, though
 * not bitwise the norm pass's own tree.  `tile_scratch` is caller-provided device
 * memory for ceil(shard_numel / 256) doubles; its contents are working storage (the
 * per-tile sums, in an internal order grouped by XCD), not an output.
 * ---------------------------------------------------------------------------- */
int32_t hbt_grad_local_share_sqnorm(const void* const* rank_grads, int32_t group_size, int32_t rank,
                                    int64_t shard_numel, int64_t valid_numel, int32_t in_dtype,
                                    int32_t reduce_dtype, float divisor, int32_t out_dtype, void* out,
                                    double* partials, double* tile_scratch, void* stream);

/* ------------------------------------------------------------------------------
 * The reduction that ends a no_sync accumulation, in one pass: hbt_grad_local_share
 * (or, with partials and tile_scratch, hbt_grad_local_share_sqnorm) where rank q's
 * element is first added to its accumulated gradient, x_q = R(cast(g_q) + a_q), R
 * rounding to the reduce dtype.
 *
 * Replaces: the final micro-batch of FlatParamHandle.reduce_scatter_gradient under
 *   no_sync, `grad = grad + self._unsharded_grad_accumulator` then the reduce-scatter
 *   (parallel/fsdp.py:747-769).
 * accumulators[q] points at row q of the accumulator: rank q's accumulated gradient
 * over this rank's slice, shard_numel elements in reduce_dtype (F32, BF16 or F16; an
 * F64 reduce dtype returns HBT_ERR_UNSUPPORTED: accumulate with hbt_grad_accumulate and
 * reduce the rows instead).  rank_grads[q] are the last micro-batch's padded full
 * gradients, read at rank * shard_numel as in hbt_grad_local_share.  The outputs are
 * bitwise those of hbt_grad_accumulate (acc = R(acc + R(grad))) over the rows followed
 * by hbt_grad_local_share_sqnorm over them at rank offset 0, which read and write every
 * row once more; NaNs included (a bf16 sum that is NaN is the canonical 0x7FC0, as the
 * accumulator stores it).  partials and tile_scratch are both given or both NULL.
 * ---------------------------------------------------------------------------- */
int32_t hbt_grad_local_share_accumulated(const void* const* rank_grads, const void* const* accumulators,
                                         int32_t group_size, int32_t rank, int64_t shard_numel, int64_t valid_numel,
                                         int32_t in_dtype, int32_t reduce_dtype, float divisor, int32_t out_dtype,
                                         void* out, double* partials, double* tile_scratch, void* stream);

/* ------------------------------------------------------------------------------
 * FSDP no_sync gradient accumulation over up to HBT_MAX_TENSORS_PER_LAUNCH
 * (accumulator, gradient) pairs.
 *
 * Replaces: the accumulate branch of FlatParamHandle.reduce_scatter_gradient
 *   (parallel/fsdp.py:733-749): grad.to(reduce_dtype), then accumulator =
 *   grad.clone() on the first micro-batch inside no_sync() and accumulator.add_(grad)
 *   on later ones, and the synchronising call's grad + accumulator before the
 *   reduce-scatter.
 * `accumulators` and `grads` are HOST arrays of `count` device addresses.  Accumulator
 * k holds numels[k] elements of acc_dtype (the reduce dtype); gradient k as many of
 * grad_dtype (each F32, BF16 or F16).  With R rounding to acc_dtype (round to nearest
 * even; the identity for F32), each element becomes
 *   acc = R(grad)                    with HBT_ACCUMULATE_ASSIGN (the clone; no read of acc)
 *   acc = R(acc + R(grad))           otherwise (the sum computed in fp32, rounded once)
 * where R(grad) is the cast (none when the dtypes match).  An F64 accumulator (reduce
 * dtype float64) takes F64 gradients too and adds in double: acc = acc + double(grad).
 * A gradient must not overlap its accumulator.
 * ---------------------------------------------------------------------------- */
#define HBT_ACCUMULATE_ASSIGN 1
int32_t hbt_grad_accumulate(void* const* accumulators, const void* const* grads, const int64_t* numels,
                            int32_t count, int32_t acc_dtype, int32_t grad_dtype, int32_t flags, void* stream);

/* ------------------------------------------------------------------------------
 * In-place gradient scaling: x = (x * unscale) * (*grad_mul), each product rounded to
 * the tensor's dtype (F32, BF16 or F16), over up to HBT_MAX_TENSORS_PER_LAUNCH tensors.
 *
 * Replaces: the grad.mul_(inverse) loop of GradScaler.unscale_
 *   (optim/grad_scaler.py:181-186) and the grad.mul_(clip_coefficient) loop of
 *   ShardedOptimizer.clip_grad_norm (optim/sharded_optimizer.py:333-337).  The fused
 *   optimizer path folds both multiplies into hbt_adamw_step instead; this entry
 *   point materialises them when a caller needs the scaled gradients themselves.
 * grad_mul may be NULL (treated as 1).  When unscale == 1 and *grad_mul == 1 nothing is
 * read or written: the reference multiplies only when its clip coefficient is below 1,
 * so the gradient keeps its bits (a bf16 NaN payload included).
 * ---------------------------------------------------------------------------- */
int32_t hbt_scale_inplace(void* const* tensors, const int64_t* numels, int32_t count,
                          int32_t dtype, float unscale, const float* grad_mul, void* stream);

/* ------------------------------------------------------------------------------
 * In-place unscale fused with its overflow check: x = R(x * unscale) (dtype F32, BF16
 * or F16, over up to HBT_MAX_TENSORS_PER_LAUNCH tensors), and in the same pass the
 * squared-norm partials of the result, weight 1.
 *
 * Replaces: the grad.mul_(inverse) loop of GradScaler.unscale_
 *   (optim/grad_scaler.py:181-186) followed by its finiteness check,
 *   GradScaler._detect_non_finite (optim/grad_scaler.py:189-200).
 * Writes exactly what hbt_scale_inplace(tensors, numels, count, dtype, unscale, NULL)
 * writes, and exactly the partials hbt_grad_sqnorm_partials then computes over the
 * scaled tensors with weights 1 and unscale 1 (hbt_norm_partials_count of them): the
 * same per-chunk order, so hbt_grad_norm_finalize gives the overflow flag, and the same
 * partials serve a later norm of the unchanged gradients.  Reads and writes each
 * element once, where the two calls read it twice.  With unscale == 1 nothing is
 * written and only the partials are computed.
 * For BF16 and F16, piece_scratch is caller-provided device memory for
 * 128 * hbt_norm_partials_count(numels, count, dtype) doubles (working storage: the sums
 * of 512-element pieces, in an internal order grouped by XCD); it may be NULL for F32 or
 * when unscale == 1.  The partials of 2-byte gradients, here and in
 * hbt_grad_sqnorm_partials, are summed per piece (a butterfly over 64 lanes of 8-element
 * lane sums) and then per chunk (a butterfly of s_l + s_(l+64)), so both passes agree.
 * ---------------------------------------------------------------------------- */
int32_t hbt_scale_inplace_sqnorm(void* const* tensors, const int64_t* numels, int32_t count,
                                 int32_t dtype, float unscale, double* partials, double* piece_scratch,
                                 void* stream);

/* ------------------------------------------------------------------------------
 * Float64 parameters: the fused clip + AdamW step, the fused clip + SGD step and the
 * in-place gradient scaling on float64 tensors, with double scalars.
 *
 * Replaces: the same reference lines as hbt_adamw_step, hbt_sgd_step and hbt_scale_inplace,
 *   for the float64 masters the reference steps when mixed precision is off and the
 *   parameters are float64 (parallel/fsdp.py:379-393; config.py:55-56 accepts "float64"),
 *   and torch.optim.AdamW / SGD on float64 tensors (optim/sharded_optimizer.py:111-126).
 * On float64 tensors torch uses every Python scalar as the double it is, so these take
 * double scalars and compute in double: per element, the op sequences documented for
 * hbt_adamw_step and hbt_sgd_step with R_G and R_P the identity, each operation one
 * correctly rounded double result (fma fused), sqrt and the divisions correctly rounded.
 * The host computes the scalars as torch does (decay = 1 - lr*wd, lerp_weight = 1 - beta1,
 * bias_correction2_sqrt = (1 - beta2^step)^0.5, neg_step_size = -lr / (1 - beta1^step);
 * for SGD the unrounded alphas).  grad_mul: the double clip multiplier
 * (hbt_grad_norm_finalize's grad_mul64_out) or NULL for 1.  flags as for hbt_adamw_step /
 * hbt_sgd_step.  hbt_scale_inplace_f64 multiplies x = (x * unscale) * (*grad_mul), each
 * product rounded in double, and reads and writes nothing when both factors are 1.
 * ---------------------------------------------------------------------------- */
int32_t hbt_adamw_step_f64(double* const* params, double* const* grads, double* const* exp_avgs,
                           double* const* exp_avg_sqs, const int64_t* numels, int32_t count, double unscale,
                           const double* grad_mul, double decay, double lerp_weight, double beta2,
                           double one_minus_beta2, double bias_correction2_sqrt, double eps, double neg_step_size,
                           int32_t flags, void* stream);
int32_t hbt_sgd_step_f64(double* const* params, double* const* grads, double* const* momentum_buffers,
                         const int64_t* numels, int32_t count, double unscale, const double* grad_mul,
                         double weight_decay, double momentum, double one_minus_dampening, double neg_lr,
                         int32_t flags, void* stream);
int32_t hbt_scale_inplace_f64(double* const* tensors, const int64_t* numels, int32_t count, double unscale,
                              const double* grad_mul, void* stream);

/* ------------------------------------------------------------------------------
 * The optimizer steps with their scalars read from device memory, for a step recorded
 * once into a HIP graph and replayed.
 *
 * Replaces: the same reference step as hbt_adamw_step, hbt_sgd_step and their float64
 *   forms (ShardedOptimizer.step, optim/sharded_optimizer.py:340-355, running
 *   torch.optim.AdamW / SGD built at optim/sharded_optimizer.py:111-126), whose host
 *   recomputes the bias corrections (torch/optim/adam.py) every step.
 * A launch recorded into a graph keeps the scalar arguments it was recorded with, while
 * AdamW's bias corrections change every step, and every scalar changes with the
 * learning rate.  Each *_slot entry point takes the arguments of its eager form plus
 * `slot`, HBT_STEP_SLOT_BYTES of 16-byte-aligned device memory; its kernels read their
 * scalars from the slot when they run, not from the arguments.  The arguments still
 * choose the kernel variant (unscale != 1; |lerp_weight| < 0.5 for AdamW; the flags) and
 * are validated as by the eager form.  Each *_write_scalars call writes into a slot, by
 * one launch on `stream`, exactly the scalars the eager form passes its kernels for the
 * same arguments (for SGD, the flags' weight-decay and Nesterov bits).  Written on the
 * replay's stream before each replay, they make the recorded step the eager step those
 * arguments describe, bit for bit.  The values written must keep the variant that the
 * step was recorded with, and the writer must match the step it feeds: AdamW or SGD,
 * float64 or not, and the same param_dtype.
 * ---------------------------------------------------------------------------- */
#define HBT_STEP_SLOT_BYTES 128
int32_t hbt_adamw_step_slot(void* const* params, void* const* grads, void* const* exp_avgs,
                            void* const* exp_avg_sqs, const int64_t* numels, int32_t count,
                            int32_t param_dtype, int32_t grad_dtype, float unscale, const float* grad_mul,
                            float decay, float lerp_weight, float beta2, float one_minus_beta2,
                            float bias_correction2_sqrt, float eps, float neg_step_size, const void* slot,
                            int32_t flags, void* stream);
int32_t hbt_adamw_write_scalars(void* slot, int32_t param_dtype, float unscale, float decay, float lerp_weight,
                                float beta2, float one_minus_beta2, float bias_correction2_sqrt, float eps,
                                float neg_step_size, void* stream);
int32_t hbt_sgd_step_slot(void* const* params, void* const* grads, void* const* momentum_buffers,
                          const int64_t* numels, int32_t count, int32_t param_dtype, int32_t grad_dtype,
                          float unscale, const float* grad_mul, float weight_decay, float momentum,
                          float one_minus_dampening, float neg_lr, const void* slot, int32_t flags, void* stream);
int32_t hbt_sgd_write_scalars(void* slot, int32_t param_dtype, float unscale, float weight_decay, float momentum,
                              float one_minus_dampening, float neg_lr, int32_t flags, void* stream);
int32_t hbt_adamw_step_f64_slot(double* const* params, double* const* grads, double* const* exp_avgs,
                                double* const* exp_avg_sqs, const int64_t* numels, int32_t count, double unscale,
                                const double* grad_mul, double decay, double lerp_weight, double beta2,
                                double one_minus_beta2, double bias_correction2_sqrt, double eps,
                                double neg_step_size, const void* slot, int32_t flags, void* stream);
int32_t hbt_adamw_write_scalars_f64(void* slot, double unscale, double decay, double lerp_weight, double beta2,
                                    double one_minus_beta2, double bias_correction2_sqrt, double eps,
                                    double neg_step_size, void* stream);
int32_t hbt_sgd_step_f64_slot(double* const* params, double* const* grads, double* const* momentum_buffers,
                              const int64_t* numels, int32_t count, double unscale, const double* grad_mul,
                              double weight_decay, double momentum, double one_minus_dampening, double neg_lr,
                              const void* slot, int32_t flags, void* stream);
int32_t hbt_sgd_write_scalars_f64(void* slot, double unscale, double weight_decay, double momentum,
                                  double one_minus_dampening, double neg_lr, int32_t flags, void* stream);

/* ------------------------------------------------------------------------------
 * The step scalars formatted on the host, for writing several slots at once.
 *
 * Replaces: the same reference step as the *_write_scalars entry points above
 *   (ShardedOptimizer.step, optim/sharded_optimizer.py:340-355).
 * Each *_scalar_record call validates its arguments as the *_write_scalars form with the
 * same name does and writes into `record`, HBT_STEP_SLOT_BYTES of host memory, the
 * bytes that form would write into a slot (zero past the scalars), launching nothing.
 * A caller holding the records of consecutive slots writes them with one
 * hbt_write_words call: a replay of several recorded steps then issues one launch for
 * their scalars instead of one per step.
 * ---------------------------------------------------------------------------- */
int32_t hbt_adamw_scalar_record(void* record, int32_t param_dtype, float unscale, float decay, float lerp_weight,
                                float beta2, float one_minus_beta2, float bias_correction2_sqrt, float eps,
                                float neg_step_size);
int32_t hbt_sgd_scalar_record(void* record, int32_t param_dtype, float unscale, float weight_decay, float momentum,
                              float one_minus_dampening, float neg_lr, int32_t flags);
int32_t hbt_adamw_scalar_record_f64(void* record, double unscale, double decay, double lerp_weight, double beta2,
                                    double one_minus_beta2, double bias_correction2_sqrt, double eps,
                                    double neg_step_size);
int32_t hbt_sgd_scalar_record_f64(void* record, double unscale, double weight_decay, double momentum,
                                  double one_minus_dampening, double neg_lr, int32_t flags);

/* ------------------------------------------------------------------------------
 * Small host-built data written into device memory by kernel launches.
 *
 * This entry point has no counterpart in the reference.  It is for callers that record
 * work into a HIP graph: a copy from pageable host memory cannot be recorded, and a
 * recorded copy from pinned memory reads that memory at every replay.  It writes
 * words[0 .. count) to `dst` (4-byte-aligned device memory) by launches on `stream` of
 * at most 256 words each; the words travel in the launch arguments, so a recorded launch
 * keeps them and the host buffer may be reused as soon as the call returns.  Used for
 * the interval tables of copies recorded into a graph, and for the step slots of a
 * recorded step before each replay.
 * ---------------------------------------------------------------------------- */
int32_t hbt_write_words(void* dst, const uint32_t* words, int64_t count, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HBT_H */
