/*
 * b3_workload.h - synthetic per-step inputs for the five benchmark scenes,
 * applied on the device.
 *
 * These are the engine-side twins of b3s_apply_inputs and b3w_masks in
 * puffysics_amd/scenes (same counter-based random numbers, same order of
 * operations), playing the part of an environment's action kernel: they
 * write forces, torques, impulses and hinge targets into the engine's live
 * worlds between b3_batch_restore_gpu and b3_batch_step_gpu.  Scene ids:
 * 1 hover, 2 box stacks, 3 hinge chains, 4 contact bin, 5 arm with free
 * bodies.  Both calls enqueue on `stream` and return hipErrorInvalidValue
 * for an unknown scene or a NULL output.
 */
#ifndef PUFFYSICS_AMD_B3_WORKLOAD_API_H
#define PUFFYSICS_AMD_B3_WORKLOAD_API_H

#include "b3_engine.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Reset and step masks of vector step `step` for worlds [0, count). */
hipError_t b3w_masks_gpu(int scene, unsigned long long seed, int step, int count, unsigned char* reset_out,
    unsigned char* step_out, hipStream_t stream);

/* Apply the scene's inputs of vector step `step` to every world selected by
 * `step_mask` (NULL = all). */
hipError_t b3w_inputs_gpu(B3Engine* engine, int scene, unsigned long long seed, int step,
    const unsigned char* step_mask, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif
