/*
 * dsa_probe.h — C ABI of libdsa_probe.so, the measurement probe bench.py
 * uses to put a measured figure beside the MI355X's published bf16 dense
 * MFMA peak (2.5 PFLOP/s).  No counterpart in the reference, which has no
 * roofline to measure against.
 */
#ifndef DSA_PROBE_H_
#define DSA_PROBE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Launches `workgroups` workgroups of 256 threads on `stream`; every wave
 * issues `iters` x 4 independent v_mfma_f32_32x32x16_bf16 (32768 flops
 * each) and writes one float per lane to `sink` (device memory of
 * workgroups * 256 floats), so that the products are not optimised away.
 * Returns 0, or nonzero if the launch failed.  Flops of the launch:
 * workgroups * 4 * iters * 4 * 32768. */
int dsa_probe_mfma_bf16(int workgroups, int iters, float* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DSA_PROBE_H_ */
