/*
 * b3_forces.hip - the engine's step with a built-in force law in the
 * per-substep force hook (B3_USER_FORCES, 01_config.inl:189-198 and
 * 09_step.inl:20-53).
 *
 * Same launch as b3k_step (one wave64 workgroup per tile of 64 worlds, one
 * world per lane, optional fused masked restore); the law runs inside the
 * lane's substep loop, before each velocity update, on the lane's own world.
 *
 *   b3k_step_gravity   Plummer-softened pairwise gravity between each
 *                      world's bodies (nbody_rigid.cuh:15-66)
 *   b3k_step_fluid     ambient-fluid forces (ambient.h:76-370) with a
 *                      per-world state array
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

/* cosf / sinf of the fluid law's golden-angle sample directions, filled
 * from the host's library when an engine is created on the device. */
__device__ float g_fluid_trig[2 * kFluidTrig];

__global__ __launch_bounds__(64) void b3k_step_fluid(uint32_t* live, const uint32_t* snap, uint32_t* scratch,
        Geometry g, int count, float dt, int substeps, const unsigned char* step_mask,
        const unsigned char* reset_mask, unsigned int opts, FluidParams law, float* state) {
    extern __shared__ float vel_rows[];
    int tile = blockIdx.x;
    int lane = threadIdx.x;
    int w = tile * 64 + lane;
    size_t words = (size_t)6 * g.max_b + 1;
    if (reset_mask) {
        restore_tile(live, snap, g, count, reset_mask, blockIdx.x, 0, 1);
        /* a restored world starts without previous velocities (b3_fluid_state_reset, ambient.h:69-74) */
        if (w < count && reset_mask[w]) state[w * words + 6 * g.max_b] = 0.0f;
        __syncthreads();
    }
    if (w >= count || (step_mask && !step_mask[w])) return;
    FluidLaw f;
    f.f = law;
    f.state = state + w * words;
    f.trig = g_fluid_trig;
    step_world(lane_view(live, scratch, vel_rows, g, tile, lane, opts), dt, substeps, f);
}

}  // namespace

/* Set-up for the force-law kernels on the current device, called by
 * b3_engine_create: their dynamic LDS limit (b3i_lds_limit) and the fluid
 * law's sample table. */
hipError_t b3i_forces_init() {
    hipError_t err;
    if ((err = b3i_lds_limit((const void*)b3k_step_gravity)) != hipSuccess) return err;
    if ((err = b3i_lds_limit((const void*)b3k_step_fluid)) != hipSuccess) return err;
    static float table[2 * kFluidTrig];
    fluid_trig_table(table);
    return hipMemcpyToSymbol(HIP_SYMBOL(g_fluid_trig), table, sizeof(table));
}

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

hipError_t b3_fluid_law_default(B3FluidLaw* out) {
    /* b3_fluid_default (ambient.h:46-60) */
    if (!out) return hipErrorInvalidValue;
    out->density = 1.2f;
    out->separation_cos = 0.0f;
    out->mu = 1.8e-5f;
    out->drag_scale = 1.0f;
    out->fric_scale = 1.0f;
    out->added_scale = 1.0f;
    out->sphere_samples = 48;
    out->box_face_samples = 3;
    out->capsule_rings = 8;
    out->buoyancy = 1;
    return hipSuccess;
}

int b3_fluid_state_words(const B3Engine* e) { return e ? 6 * e->g.max_b + 1 : -1; }

hipError_t b3_batch_step_fluid_gpu(B3Engine* e, float dt, int substeps, const unsigned char* step_mask,
        const unsigned char* reset_mask, const B3FluidLaw* law, float* state, hipStream_t stream) {
    if (!e || !law || !isfinite(dt) || dt < 0.0f || substeps < 1 || law->sphere_samples > kFluidTrig
            || law->box_face_samples > B3_FLUID_MAX_FACE_SAMPLES || law->capsule_rings > B3_FLUID_MAX_RINGS)
        return hipErrorInvalidValue;
    if (e->options & B3_ENGINE_ART_CONTACTS) return hipErrorNotSupported;
    if (e->count == 0) return hipSuccess;
    if (!state) return hipErrorInvalidValue;
    hipError_t err = on_device(e);
    if (err != hipSuccess) return err;
    if (dt == 0.0f && !reset_mask) return hipSuccess;
    FluidParams p;
    p.density = law->density;
    p.separation_cos = law->separation_cos;
    p.mu = law->mu;
    p.drag_scale = law->drag_scale;
    p.fric_scale = law->fric_scale;
    p.added_scale = law->added_scale;
    p.sphere_samples = law->sphere_samples;
    p.box_face_samples = law->box_face_samples;
    p.capsule_rings = law->capsule_rings;
    p.buoyancy = law->buoyancy;
    b3k_step_fluid<<<e->tiles, 64, e->lds_bytes, stream>>>(e->live, e->snap, e->scratch, e->g, e->count, dt,
        substeps, step_mask, reset_mask, e->options, p, state);
    return hipGetLastError();
}

}  // extern "C"
