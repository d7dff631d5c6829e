/*
 * pcp_probe.h — HBM stream probes: the practical bandwidth roof of this device.
 *
 * No counterpart in the reference (it runs the loss head inside its compiled VMFB and
 * measures nothing of the kind). Measurement infrastructure for the roofline figures:
 * the bandwidth plain streaming kernels reach for the access mixes of the library's
 * HBM-bound kernels, beside the 8 TB/s spec figure.
 */
#ifndef PCP_PROBE_H
#define PCP_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

struct pcp_ctx;

/* One stream over `bytes` (a positive multiple of 16; buffers 16-byte aligned):
 *   kind 0 read:  reads a                      (c: a 16-byte word written only if the
 *                                                  XOR of all of a is all ones)
 *   kind 1 write: writes c
 *   kind 2 copy:  c = a
 *   kind 3 mix:   c = a ^ b                    (two reads per write)
 * nontemporal != 0 uses nontemporal loads and stores. The grid is flat: each 256-lane
 * workgroup moves 256 x vectors_per_lane (1, 2, 4 or 8) 16-byte vectors. Asynchronous
 * on `stream`; timed by pcp_profile_start / pcp_profile_stop like the other entry
 * points. */
int pcp_hbm_stream(struct pcp_ctx* ctx, int kind, int nontemporal, int vectors_per_lane, const void* a,
                   const void* b, void* c, int64_t bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PCP_PROBE_H */
