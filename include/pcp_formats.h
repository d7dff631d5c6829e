/*
 * pcp_formats.h — the on-disk and wire formats around the GRPO step, read and written
 * straight from and to HBM.
 *
 *  - Prompt dataset (.bin, tools/prepare_rl_dataset.py:28-40, read by
 *    GRPO.loadPrompts, src/algorithms/grpo.zig:63-91): u32 count, then per prompt
 *    u32 length and length u64 token ids, all little-endian.
 *  - Master weights (tools/convert_weights.py:39-44, read by
 *    RLShepherd.loadWeightsFromFile, src/nodes/controllers/rl_shepherd.zig:141-229):
 *    the f32 tensors in named_parameters() order, concatenated, no header.
 *  - UPDATE_WEIGHTS payload (rl_shepherd.zig:691-711 encodes, Worker
 *    handleUpdateWeights, src/nodes/workers/worker.zig:2631-2667 decodes): the weight
 *    bytes in base64, standard alphabet with '=' padding (std.base64.standard).
 *
 * Status codes and the context are those of pcp_grpo.h.
 */
#ifndef PCP_FORMATS_H
#define PCP_FORMATS_H

#include <stdint.h>

#include "pcp_grpo.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ~ GRPO.loadPrompts. With tokens == NULL (or offsets == NULL) only *n_prompts and
 * *n_tokens are returned; otherwise the prompts are written in the layout of
 * pcp_pack_rollouts: tokens (device, int64[n_tokens], the prompts concatenated) and
 * offsets (device, int64[n_prompts + 1]); tokens_cap / offsets_cap give their sizes.
 * PCP_ERR_IO when the file cannot be read, PCP_ERR_CORRUPT_STATE when it ends inside a
 * record (the reference's EndOfStream), PCP_ERR_OVERFLOW for an id above 2^63 - 1
 * (the reference's @intCast to i64) or a buffer that is too small. */
int pcp_prompts_load(pcp_ctx* ctx, const char* path, int64_t* tokens, int64_t tokens_cap, int64_t* offsets,
                     int64_t offsets_cap, int64_t* n_prompts, int64_t* n_tokens);

/* ~ RLShepherd.loadWeightsFromFile: n_tensors tensors of counts[i] f32 elements from
 * the start of the file into one device buffer (tensor i at counts[0] + ... +
 * counts[i-1]), staged through pinned host memory with the copies overlapping the
 * reads. bf16 (device, may be NULL) receives the weights rounded to bf16 (nearest
 * even) in the same pass. PCP_ERR_CORRUPT_STATE when the file is shorter than the
 * tensors (WeightFileTooSmall); extra bytes are ignored, as in the reference. */
int pcp_weights_load(pcp_ctx* ctx, const char* path, int n_tensors, const int64_t* counts, float* dev,
                     void* bf16);
/* The inverse: n f32 elements of a device buffer to a new file (the checkpoint the
 * reference's optimizer writes back into its mapped file). */
int pcp_weights_save(pcp_ctx* ctx, const char* path, const float* dev, int64_t n);

/* Base64 (standard alphabet, '=' padding) of nbytes device bytes into dst (device,
 * pcp_base64_encoded_len(nbytes) bytes, no terminator). */
int64_t pcp_base64_encoded_len(int64_t nbytes);
int pcp_base64_encode(pcp_ctx* ctx, const void* src, int64_t nbytes, char* dst, void* stream);
/* Decodes len characters (device) into dst (device, at least len / 4 * 3 bytes);
 * *nbytes receives the decoded size. PCP_ERR_INVALID_ARG for a length that is not a
 * multiple of 4, a character outside the alphabet, misplaced padding or non-zero bits
 * below the last character of a padded quad (std.base64's InvalidPadding /
 * InvalidCharacter). */
int pcp_base64_decode(pcp_ctx* ctx, const char* src, int64_t len, void* dst, int64_t* nbytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PCP_FORMATS_H */
