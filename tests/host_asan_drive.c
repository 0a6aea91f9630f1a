// Host-only drive of libhbt's argument checks and table builders, run under AddressSanitizer by
// tests/test_host_asan.py: every entry point with tables up to and past its limits,
// empty tensors (nothing to launch) and bad arguments, no device needed.
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "hbt.h"

static int fails = 0;
#define EXPECT(cond) do { if (!(cond)) { printf("FAIL line %d: %s (%s)\n", __LINE__, #cond, hbt_last_error()); fails++; } } while (0)

int main(void) {
    static float buf[1 << 16] __attribute__((aligned(64)));  // 16-byte aligned slots
    void* ptrs[64];
    const void* cptrs[64];
    int64_t numels[64];
    double weights[64];
    for (int i = 0; i < 64; ++i) { ptrs[i] = buf + i; cptrs[i] = buf + i; numels[i] = 0; weights[i] = 1.0; }
    double partials[16];
    // version, symbols, helpers
    EXPECT(hbt_abi_version() == HBT_TEST_ABI && hbt_symbol_count() == HBT_TEST_SYMBOLS);
    for (int s = -1; s < 6; ++s) for (int d = -1; d < 6; ++d) (void)hbt_copy_chunk_elems(s, d);
    int64_t first[8], count[8];
    EXPECT(hbt_grid_slices(0, 64, first, count, 8) == 0);
    EXPECT(hbt_grid_slices(10, 0, first, count, 8) == -1);
    EXPECT(hbt_grid_slices(1LL << 40, 64, first, count, 8) > 8);  // more slices than capacity: writes 8 only
    EXPECT(hbt_grid_slices(1LL << 40, 64, NULL, NULL, 0) > 0);
    // norm partial counts and tables of every size up to and past the limit
    for (int c = -1; c <= HBT_MAX_TENSORS_PER_LAUNCH + 1; ++c) {
        (void)hbt_norm_partials_count(numels, c, HBT_DTYPE_F32);
        int rc = hbt_grad_sqnorm_partials(cptrs, numels, weights, c, HBT_DTYPE_BF16, 1.0f, partials, NULL);
        EXPECT((c >= 0 && c <= HBT_MAX_TENSORS_PER_LAUNCH) ? rc == HBT_OK : rc == HBT_ERR_INVALID_ARGUMENT);
        rc = hbt_scale_inplace(ptrs, numels, c, HBT_DTYPE_F16, 0.5f, NULL, NULL);
        EXPECT((c >= 0 && c <= HBT_MAX_TENSORS_PER_LAUNCH) ? rc == HBT_OK : rc == HBT_ERR_INVALID_ARGUMENT);
        rc = hbt_scale_inplace_sqnorm(ptrs, numels, c, HBT_DTYPE_BF16, 0.5f, partials, partials, NULL);
        EXPECT((c >= 0 && c <= HBT_MAX_TENSORS_PER_LAUNCH) ? rc == HBT_OK : rc == HBT_ERR_INVALID_ARGUMENT);
        rc = hbt_adamw_step(ptrs, ptrs, ptrs, ptrs, numels, c, HBT_DTYPE_F32, HBT_DTYPE_BF16, 1.0f, NULL,
                            1.0f, 0.1f, 0.9f, 0.1f, 1.0f, 1e-8f, -1e-3f, HBT_STEP_WRITE_GRAD, NULL);
        EXPECT((c >= 0 && c <= HBT_MAX_TENSORS_PER_LAUNCH) ? rc == HBT_OK : rc == HBT_ERR_INVALID_ARGUMENT);
        rc = hbt_sgd_step(ptrs, ptrs, ptrs, numels, c, HBT_DTYPE_F32, HBT_DTYPE_F32, 1.0f, NULL, 0.01f, 0.9f, 1.0f,
                          -0.1f, HBT_SGD_MOMENTUM, NULL);
        EXPECT((c >= 0 && c <= HBT_MAX_TENSORS_PER_LAUNCH) ? rc == HBT_OK : rc == HBT_ERR_INVALID_ARGUMENT);
        rc = hbt_grad_accumulate(ptrs, cptrs, numels, c, HBT_DTYPE_F32, HBT_DTYPE_BF16, 0, NULL);
        EXPECT((c >= 0 && c <= HBT_MAX_TENSORS_PER_LAUNCH) ? rc == HBT_OK : rc == HBT_ERR_INVALID_ARGUMENT);
    }
    // bad dtypes and pointers
    EXPECT(hbt_grad_sqnorm_partials(cptrs, numels, weights, 1, 7, 1.0f, partials, NULL) == HBT_ERR_INVALID_ARGUMENT);
    EXPECT(hbt_scale_inplace_sqnorm(ptrs, numels, 1, HBT_DTYPE_F64, 0.5f, partials, NULL, NULL) == HBT_ERR_UNSUPPORTED);
    EXPECT(hbt_scale_inplace_sqnorm(ptrs, numels, 1, HBT_DTYPE_BF16, 0.5f, partials, NULL, NULL) ==
           HBT_ERR_INVALID_ARGUMENT);  /* 2-byte gradients need the piece scratch */
    EXPECT(hbt_scale_inplace_sqnorm(ptrs, numels, 1, HBT_DTYPE_F16, 1.0f, partials, NULL, NULL) == HBT_OK);
    EXPECT(hbt_scale_inplace_sqnorm(ptrs, numels, 1, 7, 0.5f, partials, NULL, NULL) == HBT_ERR_INVALID_ARGUMENT);
    EXPECT(hbt_scale_inplace_sqnorm(ptrs, numels, 1, HBT_DTYPE_F32, 0.5f, NULL, NULL, NULL) == HBT_ERR_INVALID_ARGUMENT);
    EXPECT(hbt_scale_inplace_sqnorm(NULL, numels, 1, HBT_DTYPE_F32, 0.5f, partials, NULL, NULL) == HBT_ERR_INVALID_ARGUMENT);
    numels[0] = -1;
    EXPECT(hbt_scale_inplace_sqnorm(ptrs, numels, 1, HBT_DTYPE_F32, 0.5f, partials, NULL, NULL) == HBT_ERR_INVALID_ARGUMENT);
    numels[0] = 0;
    // local shares: every group size to the limit and past it, empty shards (no launch)
    for (int g = 0; g <= HBT_MAX_LOCAL_RANKS + 1; ++g) {
        int ok = g >= 1 && g <= HBT_MAX_LOCAL_RANKS;
        int rc = hbt_grad_local_share(cptrs, g, 0, 0, 0, HBT_DTYPE_BF16, HBT_DTYPE_F32, (float)g, HBT_DTYPE_F32,
                                      buf, NULL);
        EXPECT(ok ? rc == HBT_OK : rc == HBT_ERR_INVALID_ARGUMENT);
        rc = hbt_grad_local_share_sqnorm(cptrs, g, g > 0 ? g - 1 : 0, 0, 0, HBT_DTYPE_F16, HBT_DTYPE_BF16, 2.0f,
                                         HBT_DTYPE_BF16, buf, partials, partials, NULL);
        EXPECT(ok ? rc == HBT_OK : rc == HBT_ERR_INVALID_ARGUMENT);
        rc = hbt_grad_local_share_accumulated(cptrs, cptrs, g, 0, 0, 0, HBT_DTYPE_BF16, HBT_DTYPE_F32, 2.0f,
                                              HBT_DTYPE_F32, buf, NULL, NULL, NULL);
        EXPECT(ok ? rc == HBT_OK : rc == HBT_ERR_INVALID_ARGUMENT);
    }
    EXPECT(hbt_grad_local_share_accumulated(cptrs, NULL, 2, 0, 4, 4, HBT_DTYPE_F32, HBT_DTYPE_F32, 2.0f, HBT_DTYPE_F32,
                                            buf, NULL, NULL, NULL) == HBT_ERR_INVALID_ARGUMENT);
    EXPECT(hbt_grad_local_share_accumulated(cptrs, cptrs, 2, 0, 4, 4, HBT_DTYPE_F32, HBT_DTYPE_F32, 2.0f, HBT_DTYPE_F32,
                                            buf, partials, NULL, NULL) == HBT_ERR_INVALID_ARGUMENT);
    EXPECT(hbt_grad_local_share_accumulated(cptrs, cptrs, 2, 0, 4, 4, HBT_DTYPE_F32, HBT_DTYPE_F64, 2.0f, HBT_DTYPE_F32,
                                            buf, NULL, NULL, NULL) == HBT_ERR_UNSUPPORTED);
    EXPECT(hbt_grad_local_share(cptrs, 2, 2, 4, 4, HBT_DTYPE_F32, HBT_DTYPE_F32, 2.0f, HBT_DTYPE_F32, buf, NULL)
           == HBT_ERR_INVALID_ARGUMENT);  // rank out of range
    EXPECT(hbt_grad_local_share(cptrs, 2, 0, 4, 5, HBT_DTYPE_F32, HBT_DTYPE_F32, 2.0f, HBT_DTYPE_F32, buf, NULL)
           == HBT_ERR_INVALID_ARGUMENT);  // valid > shard
    // copy plans: refused before any device work
    EXPECT(hbt_copy_intervals(NULL, 1, 1, HBT_DTYPE_F32, HBT_DTYPE_F32, HBT_COPY_OP_COPY, 1.0f, 0, NULL)
           == HBT_ERR_INVALID_ARGUMENT);
    EXPECT(hbt_copy_intervals((const int64_t*)buf, 0, 0, HBT_DTYPE_F32, HBT_DTYPE_F32, HBT_COPY_OP_COPY, 1.0f, 0, NULL) == HBT_OK);
    EXPECT(hbt_copy_intervals((const int64_t*)buf, 1, 1, 9, HBT_DTYPE_F32, HBT_COPY_OP_COPY, 1.0f, 0, NULL) == HBT_ERR_INVALID_ARGUMENT);
    // finalize and the no-allocation norm: argument checks
    EXPECT(hbt_grad_norm_finalize(NULL, 3, 1.0, NULL, NULL, NULL, NULL, NULL, NULL) == HBT_ERR_INVALID_ARGUMENT);
    // float64 entry points: argument checks
    EXPECT(hbt_adamw_step_f64(NULL, NULL, NULL, NULL, NULL, HBT_MAX_TENSORS_PER_LAUNCH + 1, 1.0, NULL, 1.0, 0.1, 0.9,
                              0.1, 1.0, 1e-8, -1e-3, 0, NULL) == HBT_ERR_INVALID_ARGUMENT);
    EXPECT(hbt_sgd_step_f64(NULL, NULL, NULL, NULL, 0, 1.0, NULL, 0.0, 0.0, 1.0, -0.1, HBT_SGD_NESTEROV, NULL)
           == HBT_ERR_INVALID_ARGUMENT);
    EXPECT(hbt_scale_inplace_f64(NULL, NULL, 2, 1.0, NULL, NULL) == HBT_ERR_INVALID_ARGUMENT);
    EXPECT(hbt_norm_partials_count(numels, 1, HBT_DTYPE_F64) >= 0);
    EXPECT(hbt_grad_norm_noalloc(cptrs, numels, weights, HBT_MAX_TENSORS_PER_LAUNCH + 1, HBT_DTYPE_F32, 1.0f, 1.0,
                                 NULL, NULL, NULL, NULL, NULL) != HBT_OK);
    // slot forms of the steps: full tables of empty tensors launch nothing; bad slots and
    // tables are refused; the writers check slot, dtype and flags before they launch
    for (int c = 0; c <= HBT_MAX_TENSORS_PER_LAUNCH + 1; ++c) {
        int rc = hbt_adamw_step_slot(ptrs, ptrs, ptrs, ptrs, numels, c, HBT_DTYPE_BF16, HBT_DTYPE_BF16, 1.0f, NULL,
                                     1.0f, 0.1f, 0.9f, 0.1f, 1.0f, 1e-8f, -1e-3f, buf, 0, NULL);
        EXPECT(rc == (c <= HBT_MAX_TENSORS_PER_LAUNCH ? HBT_OK : HBT_ERR_INVALID_ARGUMENT));
        rc = hbt_sgd_step_slot(ptrs, ptrs, ptrs, numels, c, HBT_DTYPE_F32, HBT_DTYPE_F32, 1.0f, NULL, 0.01f, 0.9f,
                               1.0f, -0.1f, buf, HBT_SGD_MOMENTUM, NULL);
        EXPECT(rc == (c <= HBT_MAX_TENSORS_PER_LAUNCH ? HBT_OK : HBT_ERR_INVALID_ARGUMENT));
        rc = hbt_adamw_step_f64_slot((double* const*)ptrs, (double* const*)ptrs, (double* const*)ptrs,
                                     (double* const*)ptrs, numels, c, 1.0, NULL, 1.0, 0.1, 0.9, 0.1, 1.0, 1e-8, -1e-3,
                                     buf, 0, NULL);
        EXPECT(rc == (c <= HBT_MAX_TENSORS_PER_LAUNCH ? HBT_OK : HBT_ERR_INVALID_ARGUMENT));
        rc = hbt_sgd_step_f64_slot((double* const*)ptrs, (double* const*)ptrs, NULL, numels, c, 1.0, NULL, 0.0, 0.0,
                                   1.0, -0.1, buf, 0, NULL);
        EXPECT(rc == (c <= HBT_MAX_TENSORS_PER_LAUNCH ? HBT_OK : HBT_ERR_INVALID_ARGUMENT));
    }
    EXPECT(hbt_adamw_step_slot(ptrs, ptrs, ptrs, ptrs, numels, 1, HBT_DTYPE_F32, HBT_DTYPE_F32, 1.0f, NULL, 1.0f,
                               0.1f, 0.9f, 0.1f, 1.0f, 1e-8f, -1e-3f, NULL, 0, NULL) == HBT_ERR_INVALID_ARGUMENT);
    EXPECT(hbt_adamw_step_slot(ptrs, ptrs, ptrs, ptrs, numels, 1, HBT_DTYPE_F32, HBT_DTYPE_F32, 1.0f, NULL, 1.0f,
                               0.1f, 0.9f, 0.1f, 1.0f, 1e-8f, -1e-3f, (char*)buf + 4, 0, NULL)
           == HBT_ERR_INVALID_ARGUMENT);
    EXPECT(hbt_adamw_write_scalars(NULL, HBT_DTYPE_F32, 1.0f, 1.0f, 0.1f, 0.9f, 0.1f, 1.0f, 1e-8f, -1e-3f, NULL)
           == HBT_ERR_INVALID_ARGUMENT);
    EXPECT(hbt_adamw_write_scalars(buf, HBT_DTYPE_F64, 1.0f, 1.0f, 0.1f, 0.9f, 0.1f, 1.0f, 1e-8f, -1e-3f, NULL)
           == HBT_ERR_INVALID_ARGUMENT);
    EXPECT(hbt_sgd_write_scalars(buf, HBT_DTYPE_F32, 1.0f, 0.0f, 0.0f, 1.0f, -0.1f, HBT_SGD_FIRST_STEP, NULL)
           == HBT_ERR_INVALID_ARGUMENT);
    EXPECT(hbt_adamw_write_scalars_f64((char*)buf + 8, 1.0, 1.0, 0.1, 0.9, 0.1, 1.0, 1e-8, -1e-3, NULL)
           == HBT_ERR_INVALID_ARGUMENT);
    EXPECT(hbt_sgd_write_scalars_f64(buf, 1.0, 0.0, 0.0, 1.0, -0.1, 1 << 10, NULL) == HBT_ERR_INVALID_ARGUMENT);
    EXPECT(hbt_write_words(NULL, NULL, 0, NULL) == HBT_OK);
    EXPECT(hbt_write_words((char*)buf + 2, (const uint32_t*)buf, 1, NULL) == HBT_ERR_INVALID_ARGUMENT);
    EXPECT(hbt_write_words(buf, NULL, 1, NULL) == HBT_ERR_INVALID_ARGUMENT);
    /* the host formatters write exactly one slot of host memory */
    {
        unsigned char* record = (unsigned char*)malloc(HBT_STEP_SLOT_BYTES);
        EXPECT(record != NULL);
        EXPECT(hbt_adamw_scalar_record(record, HBT_DTYPE_BF16, 1.0f, 1.0f, 0.1f, 0.9f, 0.1f, 1.0f, 1e-8f, -1e-3f)
               == HBT_OK);
        EXPECT(hbt_adamw_scalar_record(record, HBT_DTYPE_F64, 1.0f, 1.0f, 0.1f, 0.9f, 0.1f, 1.0f, 1e-8f, -1e-3f)
               == HBT_ERR_INVALID_ARGUMENT);
        EXPECT(hbt_sgd_scalar_record(record, HBT_DTYPE_F16, 1.0f, 0.01f, 0.9f, 1.0f, -0.1f,
                                     HBT_SGD_MOMENTUM | HBT_SGD_NESTEROV) == HBT_OK);
        EXPECT(hbt_adamw_scalar_record_f64(record, 1.0, 1.0, 0.1, 0.9, 0.1, 1.0, 1e-8, -1e-3) == HBT_OK);
        EXPECT(hbt_sgd_scalar_record_f64(record, 1.0, 0.0, 0.0, 1.0, -0.1, HBT_SGD_WEIGHT_DECAY) == HBT_OK);
        EXPECT(hbt_sgd_scalar_record_f64(NULL, 1.0, 0.0, 0.0, 1.0, -0.1, 0) == HBT_ERR_INVALID_ARGUMENT);
        free(record);
    }
    (void)hbt_last_error();
    printf("asan host drive: %d failures\n", fails);
    return fails;
}
