/* maplesynth.h -- seeded synthetic Maple-shaped data in the reference's packed layout (csrc/synth.c).
 *
 * Bench and test tooling, built as its own library (libmaplesynth.so) beside libmaplemoe.so: it has no
 * counterpart in maple.c, which reads converted checkpoints (convert.py, layout.py). Every value is a pure
 * function of (seed, tensor id, element index), so any subset can be regenerated on the host for checking.
 */
#ifndef MAPLESYNTH_H
#define MAPLESYNTH_H
#include <stddef.h>
#include <stdint.h>

/* one expert (L, e): gate codes 512 x 512 B, gate scales 512 fp32, up the same, down codes 2048 x 128 B,
 * down scales 2048 fp32 */
void mmoe_synth_expert(uint64_t seed, int L, int e, uint8_t *gc, float *gs, uint8_t *uc, float *us, uint8_t *dc, float *ds);
/* bytes of one expert block as mmoe_synth_layer lays it out (798,720) */
size_t mmoe_synth_expert_bytes(void);
/* all 256 experts of layer L, contiguous, on nthreads host threads */
void mmoe_synth_layer(uint64_t seed, int L, uint8_t *base, int nthreads);
/* router [256][2048] bf16: dist 0 = N(0, 0.02^2), 1 = uniform (config 1) */
void mmoe_synth_router(uint64_t seed, int L, int dist, uint16_t *w);
/* nb hidden rows N(0, 1) of stream sid */
void mmoe_synth_hidden(uint64_t seed, int sid, int nb, float *x);
/* per-expert router bias log-Zipf(s) over a seeded permutation of the experts (config 2) */
void mmoe_synth_zipf_bias(uint64_t seed, double s, float *bias);

#endif
