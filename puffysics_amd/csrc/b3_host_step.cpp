/*
 * b3_host_step.cpp - the CPU step of the library: b3_step and
 * b3_batch_step on plain B3World structs in host memory.
 *
 * The reference's b3_step is a host + device function (09_step.inl:262-264)
 * and b3_batch_step its CPU loop over a B3Batch (b3_batch.cuh:39-48).  Code
 * such as a CPU environment step (puffysics_hover.h:38-56) calls them on the
 * host.  This file builds the engine's own per-lane step (b3d_lane.h) for
 * the host with B3D_LANES 1: a "tile" of one world is then exactly the
 * world's B3World bytes, its scratch and velocity rows are contiguous, and
 * the step runs in place on the caller's struct.  The arithmetic is the
 * device kernel's, so the results are the reference's bit for bit (the
 * prepared contact fields included, as the reference writes them).
 *
 * Built with g++ (-DB3D_LANES=1 -ffp-contract=off -fno-fast-math) and
 * linked into libb3engine.so; it uses no HIP call.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <vector>

#include "b3_types.h"
#include "b3d_lane.h"

static_assert(B3D_LANES == 1, "the host step is built with one world per tile");

using namespace b3d;

namespace {

/* Per-thread scratch and velocity rows, grown to the largest capacity set
 * seen; no allocation once warm. */
struct HostRows {
    std::vector<uint32_t> scratch;
    std::vector<float> vel;
};
thread_local HostRows t_rows;

int host_word(const unsigned char* world, int k) {
    int v;
    memcpy(&v, world + (size_t)k * 4, 4);
    return v;
}

/* Counts within the capacities and every body / shape index in range: the
 * conditions under which the step's indices stay inside the struct. */
bool world_in_range(const unsigned char* wp, const Geometry& g) {
    int nb = host_word(wp, H_BODY_COUNT), ns = host_word(wp, H_SHAPE_COUNT);
    int nc = host_word(wp, H_CONTACT_COUNT), nj = host_word(wp, H_JOINT_COUNT);
    if (nb < 0 || nb > g.max_b || ns < 0 || ns > g.max_s || nc < 0 || nc > g.max_c || nj < 0 || nj > g.max_j)
        return false;
    for (int s = 0; s < ns; s++) {
        int b = host_word(wp, g.so + s * kShapeWords + S_BODY);
        if (b < 0 || b >= nb) return false;
    }
    for (int j = 0; j < nj; j++) {
        int a = host_word(wp, g.jo + j * kJointWords + J_BODY_A);
        int b = host_word(wp, g.jo + j * kJointWords + J_BODY_B);
        if (a < 0 || a >= nb || b < 0 || b >= nb) return false;
    }
    for (int c = 0; c < nc; c++) {
        int base = g.co + c * kContactWords;
        int sa = host_word(wp, base + C_SHAPE_A), sb = host_word(wp, base + C_SHAPE_B);
        int ba = host_word(wp, base + C_BODY_A), bb = host_word(wp, base + C_BODY_B);
        int pc = host_word(wp, base + C_POINT_COUNT);
        if (sa < 0 || sa >= ns || sb < 0 || sb >= ns || ba < 0 || ba >= nb || bb < 0 || bb >= nb || pc < 0
                || pc > kMaxManifold)
            return false;
    }
    return true;
}

void step_one(uint32_t* world, const Geometry& g, float dt, int substeps) {
    HostRows& r = t_rows;
    if (r.scratch.size() < (size_t)g.tile_scr_words) r.scratch.resize((size_t)g.tile_scr_words);
    if (r.vel.size() < (size_t)lds_rows(g)) r.vel.resize((size_t)lds_rows(g));
    step_world(lane_view(world, r.scratch.data(), r.vel.data(), g, 0, 0, kKeepSolverFields), dt, substeps);
}

}  // namespace

extern "C" {

void b3_host_step(void* world, unsigned long long config_signature, float dt, int substeps) {
    Geometry g;
    size_t world_bytes;
    if (!world || !(dt > 0.0f) || !geometry_of(config_signature, &g, &world_bytes)) return;
    if (((uintptr_t)world & 3u) || !world_in_range((const unsigned char*)world, g)) return;
    step_one((uint32_t*)world, g, dt, substeps);
}

int b3_host_batch_step(B3Batch batch, unsigned long long config_signature, float dt, int substeps,
        const unsigned char* active) {
    Geometry g;
    size_t world_bytes;
    if (!geometry_of(config_signature, &g, &world_bytes)) return 0;
    if (batch.count < 0 || !isfinite(dt) || dt < 0.0f || substeps < 1) return 0;
    if (batch.count > 0 && (!batch.data || batch.stride < world_bytes || batch.world_offset > batch.stride - world_bytes
            || (size_t)batch.count > SIZE_MAX / batch.stride))
        return 0;
    if (((uintptr_t)batch.data | batch.stride | batch.world_offset) & 3u) return 0;
    if (dt == 0.0f) return 1;
    unsigned char* base = (unsigned char*)batch.data + batch.world_offset;
    /* no partial mutation: every selected world is checked first */
    for (int i = 0; i < batch.count; i++)
        if ((!active || active[i]) && !world_in_range(base + (size_t)i * batch.stride, g)) return 0;
    for (int i = 0; i < batch.count; i++)
        if (!active || active[i]) step_one((uint32_t*)(base + (size_t)i * batch.stride), g, dt, substeps);
    return 1;
}

}  // extern "C"
