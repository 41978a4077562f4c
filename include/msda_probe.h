/*
 * msda_probe.h — device probes of the gfx950 library, for the benchmark's roofline (no
 * counterpart in the reference: RF-DETR-JAX has no on-device measurement of its own).
 */
#ifndef MSDA_PROBE_H_
#define MSDA_PROBE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * LDS read bandwidth: launches `blocks` workgroups of 256 threads on `stream`, each streaming
 * 16-byte LDS reads (ds_read_b128, contiguous 1 KB per wave instruction) `reps` times over eight
 * 1 KB blocks; writes one 32-bit word per thread to `out` (blocks * 256 words, device memory) so
 * that the reads are kept. The caller times the launch (for example with events on `stream`) and
 * divides msda_probe_lds_read_bytes(blocks, reps) by the time. Returns 0, -1 on a bad argument,
 * -3 on a launch failure.
 */
int msda_probe_lds_read(unsigned* out, int blocks, int reps, void* stream);

/* Bytes of LDS the probe reads for (blocks, reps): blocks * 256 threads * reps * 8 reads * 16 B. */
int64_t msda_probe_lds_read_bytes(int blocks, int reps);

/*
 * LDS f64 atomic-add rate (the grad_value accumulation of msda_bwd adds with ds_add_f64):
 * launches `blocks` workgroups of 256 threads on `stream`; every thread adds 1.0 with ds_add_f64
 * 16 * reps times, each wave instruction to 64 consecutive doubles (every bank pair, each address
 * once), and writes the sum of 16 of its workgroup's accumulators to `out` (blocks * 256
 * doubles, device memory; they total 256 * 16 * reps per workgroup). The caller times the launch
 * and divides msda_probe_lds_atomic_ops(blocks, reps) by the time. Returns 0, -1 on a bad
 * argument, -3 on a launch failure.
 */
int msda_probe_lds_atomic(double* out, int blocks, int reps, void* stream);

/* Lane additions the atomic probe performs for (blocks, reps): blocks * 256 * reps * 16. */
int64_t msda_probe_lds_atomic_ops(int blocks, int reps);

/*
 * LDS f32 atomic-add rate: as msda_probe_lds_atomic with 32-bit floats (ds_add_f32 through an LDS
 * pointer; each wave instruction on 64 consecutive floats); writes blocks * 256 floats to `out`
 * (they total 256 * 16 * reps per workgroup, exact in f32 while that is below 2^24). The lane
 * additions are msda_probe_lds_atomic_ops(blocks, reps). Returns 0, -1 on a bad argument, -3 on a
 * launch failure.
 */
int msda_probe_lds_atomic_f32(float* out, int blocks, int reps, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MSDA_PROBE_H_ */
