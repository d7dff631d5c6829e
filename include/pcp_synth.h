/*
 * pcp_synth.h — seeded synthetic inputs for the GRPO loss head, generated in HBM.
 *
 * No counterpart in the reference: PCP feeds logits produced by its Qwen forward
 * pass. These functions produce inputs of the benchmark configurations directly
 * on the GPU (the full-size logit tensors are 10-20 GB each) for the benchmark
 * and the parity tests. Counter-based: every element depends only on
 * (seed, tensor tag, element index), via Philox4x32-10 (Salmon, Moraes, Dror,
 * Shaw, "Parallel random numbers: as easy as 1, 2, 3", SC'11) and Box-Muller.
 *
 * All functions are stream-ordered (stream NULL => default stream) and return
 * 0 or a negative pcp_status (pcp_grpo.h).
 */
#ifndef PCP_SYNTH_H
#define PCP_SYNTH_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Philox4x32-10 of counter (c0..c3) and key (k0, k1) on the host; out[4].
 * Exposed so tests can pin the device generator against known-answer vectors. */
void pcp_synth_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);

/* policy[i] = round(std_p * z(seed, tag 1, i));
 * ref[i]    = round(float(policy[i]) + std_r * z(seed, tag 2, i))   (ref may be NULL)
 * dtype: 1 (bf16), 0 (f16) or 2 (f32) as pcp_dtype; n elements each. */
int pcp_synth_logits(void* policy, void* ref, int64_t n, int dtype, float std_p, float std_r,
                     uint64_t seed, void* stream);

/* Gumbel-max draw of one token per row from softmax(logits[row, :]):
 * ids[row] = argmax_v ( x[row, v] - log(-log u(seed, tag 3, row*V + v)) ),
 * ties to the lowest index. ids is int64 [nrows]. */
int pcp_synth_sample_tokens(const void* logits, int dtype, int64_t nrows, int64_t vocab,
                            uint64_t seed, int64_t* ids, void* stream);

/* Target ids for the fused LM-head configuration (config 5): one token per hidden row
 * drawn from softmax(hidden[row, :] . weight^T) by Gumbel-max, as
 * pcp_synth_sample_tokens draws from given logits. The logits are formed in f32 with the
 * library's bf16 MFMA tile kernel, `chunk` rows at a time in ctx's work buffer
 * (chunk * vocab * 4 bytes; chunk 0 => 1024), and chunk k is drawn with seed + k.
 * hidden [n, hidden_dim] and weight [vocab, hidden_dim] bf16, row-major and 16-byte
 * aligned; hidden_dim a positive multiple of 64. ids is int64 [n]. */
struct pcp_ctx;
int pcp_synth_lmhead_tokens(struct pcp_ctx* ctx, const void* hidden, const void* weight, int64_t n,
                            int64_t hidden_dim, int64_t vocab, int64_t chunk, uint64_t seed, int64_t* ids,
                            void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PCP_SYNTH_H */
