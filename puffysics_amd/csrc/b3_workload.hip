/*
 * b3_workload.hip - device-side per-step inputs of the benchmark scenes.
 *
 * One lane per world, one wave per 64-world tile.  Each lane reproduces
 * b3s_apply_inputs (puffysics_amd/scenes/b3_scenes.h) on its world's
 * transposed words: the same random draws (b3s_* counter hashes, shared with
 * the host through b3_scenes.h) and the same float operations in the same
 * order, so a world stepped on the GPU sees bit-identical inputs to one
 * stepped by a host loop.
 */
#include <hip/hip_runtime.h>

#include "b3_engine_internal.h"
#include "b3_workload.h"
#include "b3d_inputs.h"

using namespace b3d;

namespace {

__global__ __launch_bounds__(64) void b3k_masks(int scene, unsigned long long seed, int step, int count,
        unsigned char* reset_out, unsigned char* step_out) {
    int w = blockIdx.x * 64 + threadIdx.x;
    if (w >= count) return;
    if (scene == B3S_ARM) {
        reset_out[w] = b3s_arm_reset(seed, w, step);
        step_out[w] = b3s_arm_step(seed, w, step);
    } else {
        reset_out[w] = 0;
        step_out[w] = 1;
    }
}

__global__ __launch_bounds__(64) void b3k_inputs(uint32_t* live, Geometry g, int count, int scene,
        unsigned long long seed, int step, const unsigned char* step_mask) {
    int tile = blockIdx.x;
    int lane = threadIdx.x;
    int w = tile * 64 + lane;
    if (w >= count || (step_mask && !step_mask[w])) return;
    Lane L;
    L.w = live + (size_t)tile * g.world_words * 64 + lane;
    L.g = g;
    scene_inputs(L, scene, seed, w, step);
}

}  // namespace

extern "C" {

hipError_t b3w_masks_gpu(int scene, unsigned long long seed, int step, int count, unsigned char* reset_out,
        unsigned char* step_out, hipStream_t stream) {
    if (scene < B3S_HOVER || scene > B3S_ARM || count < 0 || (count && (!reset_out || !step_out)))
        return hipErrorInvalidValue;
    if (count == 0) return hipSuccess;
    b3k_masks<<<(count + 63) / 64, 64, 0, stream>>>(scene, seed, step, count, reset_out, step_out);
    return hipGetLastError();
}

hipError_t b3w_inputs_gpu(B3Engine* e, int scene, unsigned long long seed, int step, const unsigned char* step_mask,
        hipStream_t stream) {
    if (!e || scene < B3S_HOVER || scene > B3S_ARM) return hipErrorInvalidValue;
    if (e->count == 0) return hipSuccess;
    b3k_inputs<<<e->tiles, 64, 0, stream>>>(e->live, e->g, e->count, scene, seed, step, step_mask);
    return hipGetLastError();
}

}  // extern "C"
