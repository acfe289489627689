/*
 * b3_forces.hip - the engine's step with the built-in force law in the
 * per-substep force hook (B3_USER_FORCES, 01_config.inl:189-198 and
 * 09_step.inl:20-53).
 *
 * Same launch as b3k_step (one wave64 workgroup per tile of 64 worlds, one
 * world per lane, optional fused masked restore); the law runs inside the
 * lane's substep loop, before each velocity update, on the lane's own world.
 *
 *   b3k_step_gravity   Plummer-softened pairwise gravity between each
 *                      world's bodies (nbody_rigid.cuh:15-66)
 */
#include <hip/hip_runtime.h>

#include <math.h>

#include "b3_engine.h"
#include "b3_engine_internal.h"
#include "b3d_forces.h"

using namespace b3d;

namespace {

__global__ __launch_bounds__(64) void b3k_step_gravity(uint32_t* live, const uint32_t* snap, uint32_t* scratch,
        Geometry g, int count, float dt, int substeps, const unsigned char* step_mask,
        const unsigned char* reset_mask, unsigned int opts, B3GravityLaw law, const float* masses) {
    extern __shared__ float vel_rows[];
    if (reset_mask) {
        restore_tile(live, snap, g, count, reset_mask, blockIdx.x, 0, 1);
        __syncthreads();
    }
    int tile = blockIdx.x;
    int lane = threadIdx.x;
    int w = tile * 64 + lane;
    if (w >= count || (step_mask && !step_mask[w])) return;
    GravityLaw f;
    f.gravity = law.gravity;
    f.softening = law.softening;
    f.masses = masses ? masses + (size_t)w * g.max_b : nullptr;
    step_world(lane_view(live, scratch, vel_rows, g, tile, lane, opts), dt, substeps, f);
}

}  // namespace

/* Set-up for the force-law kernel on the current device, called by
 * b3_engine_create: its dynamic LDS limit (b3i_lds_limit). */
hipError_t b3i_forces_init() { return b3i_lds_limit((const void*)b3k_step_gravity); }

extern "C" {

hipError_t b3_batch_step_gravity_gpu(B3Engine* e, float dt, int substeps, const unsigned char* step_mask,
        const unsigned char* reset_mask, B3GravityLaw law, const float* masses, hipStream_t stream) {
    /* nbody_cfg_ok (nbody.cuh:44-46): gravity >= 0 and softening > 0 */
    if (!e || !isfinite(dt) || dt < 0.0f || substeps < 1 || !(law.gravity >= 0.0f) || !(law.softening > 0.0f))
        return hipErrorInvalidValue;
    if (e->options & B3_ENGINE_ART_CONTACTS) return hipErrorNotSupported;
    if (e->count == 0) return hipSuccess;
    hipError_t err = on_device(e);
    if (err != hipSuccess) return err;
    if (dt == 0.0f) return reset_mask ? b3_batch_restore_gpu(e, reset_mask, stream) : hipSuccess;
    b3k_step_gravity<<<e->tiles, 64, e->lds_bytes, stream>>>(e->live, e->snap, e->scratch, e->g, e->count, dt,
        substeps, step_mask, reset_mask, e->options, law, masses);
    return hipGetLastError();
}

}  // extern "C"
