/*
 * b3_art.hip - the engine's step with articulation-aware contacts
 * (B3_ENGINE_ART_CONTACTS; the reference's B3_ART_CONTACTS=1).
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

__global__ __launch_bounds__(64) void b3k_step_art(uint32_t* live, const uint32_t* snap, uint32_t* scratch,
        float* art_ws, Geometry g, int count, float dt, int substeps, const unsigned char* step_mask,
        const unsigned char* reset_mask, unsigned int opts) {
    extern __shared__ float vel_rows[];
    if (reset_mask) {
        restore_tile(live, snap, g, count, reset_mask);
        __syncthreads();
    }
    int tile = blockIdx.x;
    int lane = threadIdx.x;
    int w = tile * 64 + lane;
    if (w >= count || (step_mask && !step_mask[w])) return;
    float* ws = art_ws + (size_t)tile * art_ws_words(g.max_b) * 64 + lane;
    step_world_art(lane_view(live, scratch, vel_rows, g, tile, lane, opts), ws, dt, substeps);
}

}  // namespace

/* The articulated step's device memory and launch limits: called by
 * b3_engine_set_options when the option is first turned on. */
hipError_t b3i_art_init(B3Engine* e) {
    hipError_t err;
    if (e->lds_bytes > 64u * 1024u) {
        err = hipFuncSetAttribute((const void*)b3k_step_art, hipFuncAttributeMaxDynamicSharedMemorySize,
            (int)e->lds_bytes);
        if (err != hipSuccess) return err;
    }
    if (e->art_ws || e->tiles == 0) return hipSuccess;
    size_t bytes = (size_t)e->tiles * art_ws_words(e->g.max_b) * 64 * sizeof(float);
    return hipMalloc((void**)&e->art_ws, bytes);
}

hipError_t b3i_step_art(B3Engine* e, float dt, int substeps, const unsigned char* step_mask,
        const unsigned char* reset_mask, hipStream_t stream) {
    b3k_step_art<<<e->tiles, 64, e->lds_bytes, stream>>>(e->live, e->snap, e->scratch, e->art_ws, e->g, e->count,
        dt, substeps, step_mask, reset_mask, e->options);
    return hipGetLastError();
}
