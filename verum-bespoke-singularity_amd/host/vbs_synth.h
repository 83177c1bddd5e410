/* vbs_synth.h — deterministic synthetic weights and activations in native
 * GGUF block layout, drawn from the distributions the benchmark configs name.
 *
 * Every block is generated from its own counter-seeded stream
 * (seed, stream, block index), so any range of blocks can be produced in
 * parallel, on any machine, with identical bytes.
 *
 *   Q4_0  d = f16(|N|*0.02),  nibbles U{0..15}
 *   Q4_1  d = f16(|N|*0.01),  m = f16(N*0.01), nibbles U{0..15}
 *   Q8_0  d = f16(|N|*0.01),  q U{-127..127}
 *   Q4_K  d, dmin = f16(|N|*0.01), 8 x (scale, min) U{0..63}, nibbles U{0..15}
 *   Q6_K  d = f16(|N|*0.01),  int8 scales U{-32..31}, 6-bit quants U{0..63}
 *   F32   N(0,1) * scale + offset
 *   F16   f16(N(0,1) * scale)
 */
#ifndef VBS_SYNTH_H
#define VBS_SYNTH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Writes n_blocks blocks of `type` (block index first_block ...) to out.
 * Returns 1 on success, 0 for a type without a generator. */
int vbs_synth_blocks(int type, uint64_t seed, uint64_t stream, uint64_t first_block,
                     uint64_t n_blocks, void *out, int nthreads);

/* out[i] = offset + scale * N(0,1), element i of stream (seed, stream). */
void vbs_synth_normal_f32(uint64_t seed, uint64_t stream, uint64_t first, size_t n,
                          float scale, float offset, float *out, int nthreads);

/* out[i] = f16(scale * N(0,1)) with the reference rounding. */
void vbs_synth_normal_f16(uint64_t seed, uint64_t stream, uint64_t first, size_t n,
                          float scale, uint16_t *out, int nthreads);

/* n token ids uniform in [0, vocab). */
void vbs_synth_tokens(uint64_t seed, uint64_t stream, uint32_t vocab, size_t n, uint32_t *out);

#ifdef __cplusplus
}
#endif
#endif
