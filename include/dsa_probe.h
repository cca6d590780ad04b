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

/* The fp32 atomic traffic that a backward without its dS workspace would
 * make to reduce the relative-table gradients over the batch: B * H * L / 128
 * workgroups, one per (b, h, 128-key tile), each adding one row of 64 floats
 * per kind (2) and per offset its keys meet (L + 127 of them) into
 * `acc`, device memory of H * 2 * (2 L) * 64 floats (zero it first; every
 * element receives a count of ones).  L a multiple of 128.  Bytes added:
 * B * H * (L / 128) * 2 * (L + 127) * 256.  Returns 0, or nonzero for bad
 * arguments or a failed launch.  No counterpart in the reference. */
int dsa_probe_dsfree_flush(int B, int H, int L, float* acc, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DSA_PROBE_H_ */
