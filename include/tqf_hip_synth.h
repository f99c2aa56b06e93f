/*
 * tqf_hip_synth.h -- synthetic workload generation for the HIP backend.
 *
 * No counterpart in the reference: its benchmarks load real checkpoints,
 * while the MI355X configurations are defined on seeded synthetic weights.
 * Generating the 18 GB resident set on the device avoids minutes of host
 * generation and PCIe transfer.  The byte definition is in
 * turboqwenfare_amd/csrc/tqf_synth.hip and is mirrored on the host by
 * turboqwenfare_amd/synth.py.
 */
#ifndef TQF_HIP_SYNTH_H
#define TQF_HIP_SYNTH_H

#include "tqf_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Nibble recipes of the synthetic Q4_0 bytes. */
#define TQF_HIP_SYNTH_UNIFORM 0u   /* nibbles uniform on 0..15 (E[q - 8] = -0.5) */
#define TQF_HIP_SYNTH_ZERO_MEAN 1u /* the same stream with nibble 0 -> 8: q - 8 on [-7, 7], mean 0 */

/* Allocates a rows x cols Q4_0 matrix and fills it with the seeded synthetic
 * bytes of (tensor_id, seed): nibbles uniform on 0..15, scales uniform on
 * [0.005, 0.02) stored as binary16. */
int32_t tqf_hip_weights_synth(tqf_hip_ctx *ctx, uint32_t rows, uint32_t cols, uint32_t tensor_id,
                              uint32_t seed, tqf_hip_weights **out);

/* The same with a nibble recipe (TQF_HIP_SYNTH_*); recipe UNIFORM gives the
 * bytes of tqf_hip_weights_synth.  An unknown recipe is TQF_HIP_ERR_INVALID. */
int32_t tqf_hip_weights_synth_recipe(tqf_hip_ctx *ctx, uint32_t rows, uint32_t cols,
                                     uint32_t tensor_id, uint32_t seed, uint32_t recipe,
                                     tqf_hip_weights **out);

#ifdef __cplusplus
}
#endif
#endif /* TQF_HIP_SYNTH_H */
