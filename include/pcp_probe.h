/*
 * pcp_probe.h — HBM stream and MFMA probes: the practical roofs of this device.
 *
 * No counterpart in the reference (it runs the loss head inside its compiled VMFB and
 * measures nothing of the kind). Measurement infrastructure for the roofline figures:
 * the bandwidth plain streaming kernels reach for the access mixes of the library's
 * HBM-bound kernels, beside the 8 TB/s spec figure, and the bf16 MFMA rate and clock
 * reached without memory traffic, beside the 2.5 PFLOP/s spec figure.
 */
#ifndef PCP_PROBE_H
#define PCP_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

struct pcp_ctx;

/* One stream over `bytes` (a positive multiple of 16; buffers 16-byte aligned):
 *   kind 0 read:  reads a                      (c: a 16-byte word written only by a lane
 *                                                  whose XOR over its own vectors is all
 *                                                  ones, which keeps the loads live)
 *   kind 1 write: writes c
 *   kind 2 copy:  c = a
 *   kind 3 mix:   c = a ^ b                    (two reads per write)
 * nontemporal != 0 uses nontemporal loads and stores. The grid is flat: each 256-lane
 * workgroup moves 256 x vectors_per_lane (1, 2, 4 or 8) 16-byte vectors, and the grid
 * must stay under 2^32 lanes (bytes / (16 * vectors_per_lane), rounded up to 256,
 * < 2^32; else PCP_ERR_INVALID_ARG). Asynchronous
 * on `stream`; timed by pcp_profile_start / pcp_profile_stop like the other entry
 * points. */
int pcp_hbm_stream(struct pcp_ctx* ctx, int kind, int nontemporal, int vectors_per_lane, const void* a,
                   const void* b, void* c, int64_t bytes, void* stream);

/* The MFMA probe: `workgroups` workgroups of 8 waves (two per SIMD, the LM-head tile
 * kernel's occupancy), each wave running `iters` (even, >= 2) rounds of independent bf16
 * MFMAs on register-resident operands: two sets of pseudo-random bf16 in [-1, 1) derived
 * from `seed`, taken alternately, the same on every wave. No memory traffic in the loop.
 *   shape 0: v_mfma_f32_32x32x16_bf16, 8 per round (32768 flops each; 4 A and 2 B
 *            fragments of 32 x 16 per set, element ((s*4 + i)*64 + lane)*8 + e and
 *            4096 + ((s*2 + j)*64 + lane)*8 + e). out[((i*2 + j)*16 + r)*64 + lane] is
 *            element r of block (i, j) of `lane`: column lane % 32, row 8 (r / 4) +
 *            4 (lane / 32) + r % 4 of the 32 x 32 product of A fragment i and B fragment j.
 *   shape 1: v_mfma_f32_16x16x32_bf16, 32 per round (16384 flops each; 8 A and 4 B
 *            fragments of 16 x 32 per set, element ((s*8 + i)*64 + lane)*8 + e and
 *            8192 + ((s*4 + j)*64 + lane)*8 + e). out[((i*4 + j)*4 + r)*64 + lane]:
 *            column lane % 16, row 4 (lane / 16) + r of the 16 x 16 product.
 * An A fragment lane holds row lane % 32 (shape 0) or lane % 16 (shape 1) at k = 8 (lane /
 * 32) or 8 (lane / 16) + e; a B fragment lane holds the column likewise.
 *   out:    [8192] f32 (4-byte aligned): the accumulators of workgroup 0's wave 0
 *   clocks: NULL or [workgroups][4] u64 (8-byte aligned): wave 0's s_memtime and
 *           s_memrealtime before and after its loop (start, end, start, end)
 * Asynchronous on `stream`; timed by pcp_profile_start / pcp_profile_stop. */
int pcp_mfma_peak(struct pcp_ctx* ctx, int shape, int workgroups, int iters, uint32_t seed, float* out,
                  uint64_t* clocks, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PCP_PROBE_H */
