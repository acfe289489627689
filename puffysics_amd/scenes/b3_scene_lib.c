/*
 * b3_scene_lib.c - host world builders of the benchmark scenes.
 *
 * Compiled once per scene with that scene's capacities (B3_MAX_*) and
 * B3W_SCENE, like any B3World user: worlds are built by the public
 * creation API (include/b3_setup.h), then handed to the engine.  Exports
 *   b3s_signature_<n>, b3s_world_size_<n>, b3s_build_batch_<n>,
 *   b3s_apply_inputs_batch_<n>
 */
#include <stddef.h>
#include "../../include/b3_setup.h"
#define B3S_WITH_BUILDERS 1
#include "b3_scenes.h"

#define B3L_CAT2(a, b) a##_##b
#define B3L_CAT(a, b) B3L_CAT2(a, b)

unsigned long long B3L_CAT(b3s_signature, B3W_SCENE)(void) { return B3_CONFIG_SIGNATURE; }
size_t B3L_CAT(b3s_world_size, B3W_SCENE)(void) { return sizeof(B3World); }

/* Build worlds first .. first + count - 1 into a contiguous array. */
int B3L_CAT(b3s_build_batch, B3W_SCENE)(void* worlds, int count, unsigned long long seed, int first) {
    for (int i = 0; i < count; i++)
        if (!b3s_build(B3W_SCENE, (B3World*)worlds + i, seed, first + i)) return 0;
    return 1;
}

/* Host application of step `step`'s inputs to the selected worlds. */
void B3L_CAT(b3s_apply_inputs_batch, B3W_SCENE)(void* worlds, int count, unsigned long long seed, int first,
        int step, const unsigned char* step_mask) {
    for (int i = 0; i < count; i++)
        if (!step_mask || step_mask[i]) b3s_apply_inputs(B3W_SCENE, (B3World*)worlds + i, seed, first + i, step);
}

#if B3W_SCENE == 1
/* Reset and step masks of vector step `step` for worlds [first, first +
 * count): the arm scene draws them, every other scene steps all worlds and
 * resets none (the same draws as the device's b3w_masks_gpu). */
void b3s_masks(int scene, unsigned long long seed, int first, int count, int step, unsigned char* reset,
        unsigned char* step_out) {
    for (int i = 0; i < count; i++) {
        if (scene == B3S_ARM) {
            reset[i] = b3s_arm_reset(seed, first + i, step);
            step_out[i] = b3s_arm_step(seed, first + i, step);
        } else {
            reset[i] = 0;
            step_out[i] = 1;
        }
    }
}
#endif
