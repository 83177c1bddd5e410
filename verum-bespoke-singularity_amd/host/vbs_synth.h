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

/* A synthetic llama-style model as a GGUF v3 file the reference loader reads
 * (src/vbs_gguf.c:88-213): general.architecture "llama", general.alignment
 * 32 and the llama.* keys of src/vbs_profiler.c:328-341 and
 * src/vbs_cpu.c:396-476; tensors in the plan order of src/vbs_graph.c:61-96
 * (token_embd, then per layer attn_norm, attn_q, attn_k, attn_v,
 * attn_output, ffn_norm, ffn_gate, ffn_up, ffn_down, then output_norm,
 * output). The bytes are the generator's streams used by the test and bench
 * models: token_embd stream 1, output 2, output_norm 3 (f32 N*0.1 + 1),
 * layer L matrix k (q,k,v,o,gate,up,down) 100 + 16L + k, its norms
 * 100 + 16L + 8 / + 9 (f32 N*0.1 + 1). Tensors are written in bounded
 * chunks, so a 70B-sized file needs no copy of itself in memory. */
typedef struct {
    uint32_t n_layers, hidden, ffn, n_heads, n_kv_heads, head_dim, vocab, context_length;
    float rope_theta, rms_eps;
    int embd_type, head_type;
    int wtype[7]; /* q, k, v, o, gate, up, down */
    uint64_t seed;
    int nthreads;
} vbs_synth_gguf_cfg_t;

/* Returns 1 on success; 0 with a message in err otherwise. */
int vbs_synth_write_gguf(const char *path, const vbs_synth_gguf_cfg_t *cfg, char *err, size_t cap);

#ifdef __cplusplus
}
#endif
#endif
