/*
 * gollek_hip_testing.h -- test-only export of libgollek_hip.so; not part of
 * the drop-in C ABI (include/gollek_hip.h), and the Java adapter never binds
 * it.
 *
 * The GEMV and MoE launchers pick their kernels from the shape, the type and
 * the buffers' alignment.  Several kernels also run correctly on shapes where
 * another kernel is faster and is the one picked; the parity tests use this
 * switch to run each kernel family on those shapes too.  The setting is
 * process-wide (every device and thread) and atomic.  Keys:
 *   "gemv_variant": 0 = automatic; 1 = the fp32 kernels everywhere;
 *                   3 = Q4_K with K <= 4096 always on the shared-tile
 *                   matrix-core kernel; 4 = Q8_0 / Q4_0 on the buffer->LDS
 *                   ring kernels and Q5_K / Q6_K on the fp32 kernel.
 *   "moe_variant":  0 = automatic; 1 = no matrix-core passes: all-Q4_K
 *                   experts on the v_dot4 passes, every other type on the
 *                   row kernels.
 * Unknown keys -> GOLLEK_HIP_ERR_ARG.
 */
#ifndef GOLLEK_HIP_TESTING_H
#define GOLLEK_HIP_TESTING_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int32_t gollek_hip_testing_set_option(const char *key, int64_t value, char *err, size_t err_len);

#ifdef __cplusplus
}
#endif
#endif /* GOLLEK_HIP_TESTING_H */
