/*
 * b3_art.hip - the engine's steps of the reference's B3_ART_CONTACTS=1
 * build (B3_ENGINE_ART_CONTACTS): b3_step with articulation-aware contacts,
 * and b3_art_step, the reduced-coordinate integrator.
 *
 * Same launch as b3k_step (one wave64 workgroup per tile of 64 worlds, one
 * world per lane, optional fused masked restore).  Each lane also owns a
 * workspace of art_ws_words(max_bodies) words, word-transposed across the
 * tile like the worlds, for its world's joint tree (b3d_art.h).
 */
#include <hip/hip_runtime.h>

#include <math.h>

#include "b3_engine.h"
#include "b3_engine_internal.h"
#include "b3d_art.h"

using namespace b3d;

namespace {

/* Reduced: b3_art_step (the reduced-coordinate integrator); otherwise
 * b3_step with articulated contacts. */
template <bool Reduced>
__global__ __launch_bounds__(64) void b3k_step_art(uint32_t* live, const uint32_t* snap, uint32_t* scratch,
        float* art_ws, Geometry g, int count, float dt, int substeps, const unsigned char* step_mask,
        const unsigned char* reset_mask, unsigned int opts) {
    extern __shared__ float vel_rows[];
    if (reset_mask) {
        restore_tile(live, snap, g, count, reset_mask, blockIdx.x, 0, 1);
        __syncthreads();
    }
    int tile = blockIdx.x;
    int lane = threadIdx.x;
    int w = tile * 64 + lane;
    if (w >= count || (step_mask && !step_mask[w])) return;
    float* ws = art_ws + (size_t)tile * art_ws_words(g.max_b) * 64 + lane;
    Lane L = lane_view(live, scratch, vel_rows, g, tile, lane, opts);
    if (Reduced) step_world_art_reduced(L, ws, dt, substeps);
    else step_world_art(L, ws, dt, substeps);
}

}  // namespace

/* The articulated steps' device memory and launch limits: called by
 * b3_engine_set_options when the option is first turned on. */
hipError_t b3i_art_init(B3Engine* e) {
    hipError_t err = b3i_lds_limit((const void*)b3k_step_art<false>);
    if (err == hipSuccess) err = b3i_lds_limit((const void*)b3k_step_art<true>);
    if (err != hipSuccess) return err;
    if (e->art_ws || e->tiles == 0) return hipSuccess;
    size_t bytes = (size_t)e->tiles * art_ws_words(e->g.max_b) * 64 * sizeof(float);
    return hipMalloc((void**)&e->art_ws, bytes);
}

hipError_t b3i_step_art(B3Engine* e, float dt, int substeps, const unsigned char* step_mask,
        const unsigned char* reset_mask, hipStream_t stream) {
    b3k_step_art<false><<<e->tiles, 64, e->lds_bytes, stream>>>(e->live, e->snap, e->scratch, e->art_ws, e->g,
        e->count, dt, substeps, step_mask, reset_mask, e->options);
    return hipGetLastError();
}

extern "C" hipError_t b3_batch_art_step_gpu(B3Engine* e, float dt, int substeps, const unsigned char* step_mask,
        const unsigned char* reset_mask, hipStream_t stream) {
    if (!e || !isfinite(dt) || dt < 0.0f || substeps < 1) return hipErrorInvalidValue;
    if (!(e->options & B3_ENGINE_ART_CONTACTS)) return hipErrorNotSupported;
    if (e->count == 0) return hipSuccess;
    hipError_t err = on_device(e);
    if (err != hipSuccess) return err;
    if (dt == 0.0f) return reset_mask ? b3_batch_restore_gpu(e, reset_mask, stream) : hipSuccess;
    b3k_step_art<true><<<e->tiles, 64, e->lds_bytes, stream>>>(e->live, e->snap, e->scratch, e->art_ws, e->g,
        e->count, dt, substeps, step_mask, reset_mask, e->options);
    return hipGetLastError();
}
