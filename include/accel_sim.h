/*
 * The standalone device calls of AccelEP's C API (include/accel/sim_api.h:16-37,
 * src/sim_api.cc:13-117) on one MI355X: a device handle, float32 uploads that stay in HBM,
 * C = A @ B with a host A and C and an uploaded B, and the stats serve/llama.py and
 * serve/sim.py read. Same names, argument meaning and return convention: 0 on success, 1 on
 * failure (a NULL handle from create and upload) with the message in accel_sim_last_error().
 *
 * An AccelSim holds no device of its own: every handle runs on the library's one GPU and
 * stream (include/accel_hip.h), and the counters are the library's.
 */
#ifndef ACCEL_SIM_H_
#define ACCEL_SIM_H_

#include <stdint.h>

#define ACCEL_SIM_API __attribute__((visibility("default")))

#ifdef __cplusplus
extern "C" {
#endif

typedef struct AccelSim AccelSim;
typedef struct AccelBuf AccelBuf;

/* accel_sim_create / destroy (sim_api.h:19-20, src/sim_api.cc:32-44). Create fails when no
 * gfx950 GPU can be initialised. */
ACCEL_SIM_API AccelSim* accel_sim_create(void);
ACCEL_SIM_API void accel_sim_destroy(AccelSim* sim);

/* accel_sim_upload / release (sim_api.h:22-24, src/sim_api.cc:46-75): count float32 values
 * copied to the device (a counted copy); the caller keeps data. */
ACCEL_SIM_API AccelBuf* accel_sim_upload(AccelSim* sim, const float* data, int64_t count);
ACCEL_SIM_API void accel_sim_release(AccelSim* sim, AccelBuf* buf);

/* accel_sim_matmul (sim_api.h:25-28, src/sim_api.cc:77-107): row-major c[m, n] = a[m, k] @ b
 * with b an uploaded [k, n] matrix. A goes to the device and C comes back as counted copies,
 * and the product is one accel_hip_matmul (one kernel matmul on the counters). */
ACCEL_SIM_API int accel_sim_matmul(AccelSim* sim, const float* a, int64_t m, int64_t k, AccelBuf* b, int64_t n,
                                   float* c);

/* Stats (sim_api.h:30-33, src/sim_api.cc:109-115): reset, kernel matmuls, and counted bytes
 * to the device and to the host (the accel_hip_get_stats fields of the same names). A Llama
 * forward (include/accel_llama.h) notes the reference's 7 MatMul calls per layer plus the LM
 * head, though its fused kernels make fewer launches. */
ACCEL_SIM_API void accel_sim_reset_stats(void);
ACCEL_SIM_API int64_t accel_sim_matmuls(void);
ACCEL_SIM_API int64_t accel_sim_bytes_to_device(void);
ACCEL_SIM_API int64_t accel_sim_bytes_to_host(void);

/* The last failure of this thread's accel_sim_* call; empty after a success (sim_api.h:36). */
ACCEL_SIM_API const char* accel_sim_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* ACCEL_SIM_H_ */
