/*
 * CPU oracle for the Familywise (FW) loss -- TEST INFRASTRUCTURE ONLY.
 *
 * Nothing in the product links, loads or calls this library.  Only tests/, the smoke() check in
 * __graft_entry__.py and the cpu_baseline leg of bench.py use it, as the checker of the HIP path.
 *
 * Two restatements, written from the reference's behaviour:
 *
 *  fwo_definition   -- the definition of reference_impl.py:11-35: sort each row descending, take
 *                      prefix sums S_k (fp64, sequential, descending order), f(k) = (S_k - 1)/k,
 *                      tau = max_k f(k).  The support is {z > tau} (strict), kappa its size
 *                      (fw_cpu.cpp:3-4, :96-101), which is also the smallest argmax of f.
 *  fwo_single_pass  -- the streaming CPU algorithm of src/cpu/fw_cpu.cpp:340-390 (chunk maximum,
 *                      running lower bound, compress of z > t, Newton tightening, final Newton),
 *                      written as scalar C with an OpenMP loop over rows.
 *
 * Output conventions (shared with the HIP path):
 *   H[r]      = largest float <= tau (so that, for a float x, x > H  <=>  x > tau)
 *   loss64[r] = (1 - z_y) + tau in fp64;  loss[r] = (float)loss64[r]
 *   kappa[r]  = |{j : z_j > tau}|
 *   grad[r,j] = (z_j > tau ? (float)(scale/kappa) : 0) , then grad[r,y] -= (float)scale   (fp32)
 */
#ifndef FWL_ORACLE_H
#define FWL_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* flags[r] bits written by fwo_definition (flags may be NULL):
 *   1: the first argmax of f(k) differs from |{z > tau}|  (never in exact arithmetic)
 *   2: max{k : z_(k) > f(k)} differs from |{z > tau}|     (never in exact arithmetic)  */
int fwo_definition(const float* z, const int64_t* y, int64_t N, int64_t C, double scale,
                   float* H, double* tau64, double* loss64, float* loss, int32_t* kappa,
                   float* grad, int32_t* flags, int nthreads);

/* Streaming restatement of fw_cpu.cpp's float32 path.  chunk <= 0 selects 2048 (fw_cpu.cpp:212),
 * cap_factor < 0 selects 4 (fw_cpu.cpp:213).  grad (may be NULL) is fully written (zeros included).
 * Returns the number of rows that needed the fallback (definition) solve. */
int64_t fwo_single_pass(const float* z, const int64_t* y, int64_t N, int64_t C, double scale,
                        double* loss64, int64_t* kappa, float* grad, int nthreads,
                        int64_t chunk, int64_t cap_factor);

/* Largest float <= t (fw_cpu.cpp:96-101). */
float fwo_round_down(double t);

#ifdef __cplusplus
}
#endif
#endif
