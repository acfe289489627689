/*
 * b3emu.cpp - host build of the engine's per-lane step, for logic tests.
 *
 * TEST INFRASTRUCTURE ONLY.  Compiles the same per-lane code the gfx950
 * kernels run (puffysics_amd/csrc/b3d_lane.h, b3d_inputs.h) with g++ and
 * drives it over word-transposed tiles one lane at a time, with a plain
 * array standing in for the LDS velocity rows.  Built with
 * -ffp-contract=off and glibc's atan2f it must match the oracle bit for
 * bit, which pins the tile layout, the restore ranges and every index the
 * kernels compute, on a machine without a GPU.  The engine library never
 * links this file.
 */
#include <stdlib.h>
#include <string.h>
#include <vector>

#include "b3d_art.h"
#include "b3d_forces.h"
#include "b3d_inputs.h"
#include "b3d_lane.h"

using namespace b3d;

extern "C" {

/* words per world and per tile of scratch, or 0 for a bad signature */
int emu_world_words(unsigned long long sig) {
    Geometry g;
    size_t wb;
    return geometry_of(sig, &g, &wb) ? g.world_words : 0;
}
int emu_scratch_words(unsigned long long sig) {
    Geometry g;
    size_t wb;
    return geometry_of(sig, &g, &wb) ? g.tile_scr_words : 0;
}

void emu_upload(const uint32_t* aos, int count, unsigned long long sig, uint32_t* tiles) {
    Geometry g;
    size_t wb;
    if (!geometry_of(sig, &g, &wb)) return;
    int ntiles = (count + kLanes - 1) / kLanes;
    memset(tiles, 0, (size_t)ntiles * g.world_words * kLanes * 4);
    for (int w = 0; w < count; w++)
        for (int k = 0; k < g.world_words; k++)
            tiles[((size_t)(w / kLanes) * g.world_words + k) * kLanes + w % kLanes] = aos[(size_t)w * g.world_words + k];
}

void emu_download(const uint32_t* tiles, int count, unsigned long long sig, uint32_t* aos) {
    Geometry g;
    size_t wb;
    if (!geometry_of(sig, &g, &wb)) return;
    for (int w = 0; w < count; w++)
        for (int k = 0; k < g.world_words; k++)
            aos[(size_t)w * g.world_words + k] = tiles[((size_t)(w / kLanes) * g.world_words + k) * kLanes + w % kLanes];
}

/* Masked restore from AoS snapshots (plain B3World structs), as the engine
 * keeps them. */
void emu_restore(uint32_t* tiles, const uint32_t* snap, int count, unsigned long long sig, const unsigned char* reset) {
    Geometry g;
    size_t wb;
    if (!geometry_of(sig, &g, &wb)) return;
    for (int w = 0; w < count; w++) {
        if (reset && !reset[w]) continue;
        size_t base = (size_t)(w / kLanes) * g.world_words * kLanes + w % kLanes;
        const uint32_t* src = snap + (size_t)w * g.world_words;
        int lo[3], hi[3];
        restore_ranges(g, (int)src[H_CONTACT_COUNT], lo, hi);
        for (int r = 0; r < 3; r++)
            for (int k = lo[r]; k < hi[r]; k++) tiles[base + (size_t)k * kLanes] = src[k];
    }
}

/* Step options (kKeepSolverFields by default, so that whole worlds compare
 * word for word with the oracle). */
static unsigned int g_opts = kKeepSolverFields;
void emu_set_options(unsigned int opts) { g_opts = opts; }

static Lane lane_of(uint32_t* tiles, uint32_t* scratch, float* vel, const Geometry& g, int w) {
    return lane_view(tiles, scratch, vel, g, w / kLanes, w % kLanes, g_opts);
}

/* Joint impulses in LDS for emu_step, as b3k_step<true> keeps them: -1 as
 * the device chooses (ji_fit), 0 never, 1 for every world with joints
 * (host memory has no LDS limit). */
static int g_joint_impulses = 0;
void emu_set_joint_impulses_lds(int mode) { g_joint_impulses = mode; }

/* Contact 0's row kept for the step in emu_step, as b3k_step<JI, true>
 * keeps it for worlds of at most two shapes: 0 never, 1 for every world
 * (the lane code handles any contact count). */
static int g_keep_row0 = 0;
void emu_set_keep_row0(int mode) { g_keep_row0 = mode; }

void emu_step(uint32_t* tiles, int count, unsigned long long sig, float dt, int substeps,
        const unsigned char* step_mask) {
    Geometry g;
    size_t wb;
    if (!geometry_of(sig, &g, &wb)) return;
    int ntiles = (count + kLanes - 1) / kLanes;
    bool ji = g_joint_impulses < 0 ? ji_fit(g) : (g_joint_impulses > 0 && g.max_j > 0);
    std::vector<uint32_t> scratch((size_t)ntiles * g.tile_scr_words);
    std::vector<float> vel((size_t)(ji ? ji_lds_rows(g) : lds_rows(g)) * kLanes);
    for (int w = 0; w < count; w++) {
        if (step_mask && !step_mask[w]) continue;
        Lane L = lane_of(tiles, scratch.data(), vel.data(), g, w);
        if (ji) {
            L.ji = vel.data() + (size_t)ji_word(g) * kLanes + w % kLanes;
            if (g_keep_row0) step_world<false, false, true, true>(L, dt, substeps);
            else step_world<false, false, true>(L, dt, substeps);
        } else {
            if (g_keep_row0) step_world<false, false, false, true>(L, dt, substeps);
            else step_world(L, dt, substeps);
        }
    }
}

/* emu_step through the shared-tile path of b3k_step_shared with a single
 * wave per tile: the staged narrowphase, the parallel preparation's
 * staging, the contact levels, and the level-by-level warm start and
 * sweeps (with one wave, a level's contacts in level order rather than
 * contact order, which must not change any result), with the joint rows in
 * LDS when they fit, as the device launch chooses. */
/* Joint rows in LDS for emu_step_shared: -1 as the device chooses
 * (joint_rows_fit), 0 never, 1 always (host memory has no LDS limit). */
static int g_joint_lds = -1;
void emu_set_joint_lds(int mode) { g_joint_lds = mode; }

void emu_step_shared(uint32_t* tiles, int count, unsigned long long sig, float dt, int substeps,
        const unsigned char* step_mask, int masks) {
    Geometry g;
    size_t wb;
    if (!geometry_of(sig, &g, &wb)) return;
    int ntiles = (count + kLanes - 1) / kLanes;
    std::vector<uint32_t> scratch((size_t)ntiles * g.tile_scr_words);
    int rows = shared_lds_words(g);
    if (kClipWords + 6 * g.max_s > rows) rows = kClipWords + 6 * g.max_s;
    if (lds_rows(g) + sched_words(g) > rows) rows = lds_rows(g) + sched_words(g);
    bool jl = g_joint_lds < 0 ? joint_rows_fit(g) : (g_joint_lds > 0 && g.max_j > 0);
    if (jl && joint_lds_word(g) + joint_lds_words(g) > rows) rows = joint_lds_word(g) + joint_lds_words(g);
    std::vector<float> lds((size_t)rows * kLanes);
    size_t max_cand = (size_t)g.max_s * (size_t)(g.max_s - 1) / 2;
    size_t words = max_cand * kStageWords;
    if ((size_t)stage_sched_words(g) > words) words = (size_t)stage_sched_words(g);
    size_t stage_tile = (1 + words) * kLanes;
    std::vector<uint32_t> stage((size_t)ntiles * stage_tile);
    bool use_masks = masks < 0 ? shared_masks(g) : (masks > 0 && g.max_s <= 64);
    for (int w = 0; w < count; w++) {
        if (step_mask && !step_mask[w]) continue;
        Lane L = lane_of(tiles, scratch.data(), lds.data(), g, w);
        PairStage S;
        S.p = stage.data() + (size_t)(w / kLanes) * stage_tile + w % kLanes;
        S.clip = lds.data() + w % kLanes;
        S.wave = 0;
        S.waves = 1;
        S.cwaves = 1;
        S.lds_bounds = 1;
        L.st = S;
        L.staged = true;
        if (jl) {
            L.jl = lds.data() + (size_t)joint_lds_word(g) * kLanes + w % kLanes;
            if (use_masks) step_world<true, true>(L, dt, substeps);
            else step_world<false, true>(L, dt, substeps);
        } else if (use_masks) {
            step_world<true>(L, dt, substeps);
        } else {
            step_world<false>(L, dt, substeps);
        }
    }
}

/* The shared-tile path with its idle lanes (worlds not in step_mask) run
 * too, as the device runs them: as wave 0 (step_world) and as a helper wave
 * (pair_helper, sweep_helper) with L.active false.  Returns 0 when every
 * lane passed the barriers a lane with its level count passes (find_pairs'
 * 3 or 4, step_world's 3, 2 around the first joint geometry and the
 * write-back, then 1 + levels per levelled pass: the warm start
 * and two sweeps per substep, and 3 per substep around the split velocity
 * and position updates and joint geometry, and with the joint rows in LDS
 * one per joint level in each of the two joint passes per substep), and an
 * idle lane's own count equals a helper's; otherwise -1 - the first world
 * that did not.  Idle lanes have no levels, so on the device, where every
 * lane passes 1 + the tile's largest level count per pass (and the tile's
 * largest joint level count per joint pass), all lanes meet the same
 * barriers. */
int emu_step_shared_idle(uint32_t* tiles, int count, unsigned long long sig, float dt, int substeps,
        const unsigned char* step_mask, int masks) {
    Geometry g;
    size_t wb;
    if (!geometry_of(sig, &g, &wb)) return -1;
    int ntiles = (count + kLanes - 1) / kLanes;
    std::vector<uint32_t> scratch((size_t)ntiles * g.tile_scr_words);
    int rows = shared_lds_words(g);
    if (kClipWords + 6 * g.max_s > rows) rows = kClipWords + 6 * g.max_s;
    if (lds_rows(g) + sched_words(g) > rows) rows = lds_rows(g) + sched_words(g);
    bool jl = joint_rows_fit(g);
    if (jl && joint_lds_word(g) + joint_lds_words(g) > rows) rows = joint_lds_word(g) + joint_lds_words(g);
    std::vector<float> lds((size_t)rows * kLanes);
    size_t max_cand = (size_t)g.max_s * (size_t)(g.max_s - 1) / 2;
    size_t words = max_cand * kStageWords;
    if ((size_t)stage_sched_words(g) > words) words = (size_t)stage_sched_words(g);
    size_t stage_tile = (1 + words) * kLanes;
    std::vector<uint32_t> stage((size_t)ntiles * stage_tile);
    bool use_masks = masks < 0 ? shared_masks(g) : (masks > 0 && g.max_s <= 64);
    int subs = substeps < 1 ? 1 : substeps;
    int fixed = (use_masks ? 4 : 3) + 3 + 2 + 3 * subs, passes = 1 + 2 * subs;
    for (int w = 0; w < count; w++) {
        bool active = !step_mask || step_mask[w];
        Lane L = lane_of(tiles, scratch.data(), lds.data(), g, w);
        PairStage S;
        S.p = stage.data() + (size_t)(w / kLanes) * stage_tile + w % kLanes;
        S.clip = lds.data() + w % kLanes;
        S.wave = 0;
        S.waves = 1;
        S.cwaves = 1;
        S.lds_bounds = 1;
        L.st = S;
        L.staged = true;
        L.active = active;
        if (jl) L.jl = lds.data() + (size_t)joint_lds_word(g) * kLanes + w % kLanes;
        host_barriers = 0;
        if (jl) {
            if (use_masks) step_world<true, true>(L, dt, substeps);
            else step_world<false, true>(L, dt, substeps);
        } else {
            if (use_masks) step_world<true>(L, dt, substeps);
            else step_world<false>(L, dt, substeps);
        }
        int levels = active ? sch_get(L, 0) : 0;
        int jlevels = jl && active ? jsch_get(L, 0) : 0;
        if (host_barriers != fixed + passes * (1 + levels) + 2 * subs * jlevels) return -1 - w;
        /* as a colliding helper (wave 1 of 2) and as one past the
         * colliding waves (wave 5 of 8, 4 colliding) */
        for (int h = 0; h < 2 && !active; h++) {
            host_barriers = 0;
            S.wave = h ? 5 : 1;
            S.waves = h ? 8 : 2;
            S.cwaves = h ? 4 : 2;
            L.st = S;
            if (use_masks) pair_helper<true>(L, S);
            else pair_helper<false>(L, S);
            if (jl) sweep_helper<true>(L, dt, substeps);
            else sweep_helper<false>(L, dt, substeps);
            if (host_barriers != fixed + passes) return -1 - w;
        }
    }
    return 0;
}

/* emu_step with pairwise gravity in the force hook; `masses` is NULL or
 * count * max_bodies floats. */
void emu_step_gravity(uint32_t* tiles, int count, unsigned long long sig, float dt, int substeps,
        const unsigned char* step_mask, float gravity, float softening, const float* masses) {
    Geometry g;
    size_t wb;
    if (!geometry_of(sig, &g, &wb)) return;
    int ntiles = (count + kLanes - 1) / kLanes;
    std::vector<uint32_t> scratch((size_t)ntiles * g.tile_scr_words);
    std::vector<float> vel((size_t)lds_rows(g) * kLanes);
    for (int w = 0; w < count; w++) {
        if (step_mask && !step_mask[w]) continue;
        GravityLaw law;
        law.gravity = gravity;
        law.softening = softening;
        law.masses = masses ? masses + (size_t)w * g.max_b : nullptr;
        step_world(lane_of(tiles, scratch.data(), vel.data(), g, w), dt, substeps, law);
    }
}

/* emu_step with articulated contacts (B3_ENGINE_ART_CONTACTS). */
void emu_step_art(uint32_t* tiles, int count, unsigned long long sig, float dt, int substeps,
        const unsigned char* step_mask) {
    Geometry g;
    size_t wb;
    if (!geometry_of(sig, &g, &wb)) return;
    int ntiles = (count + kLanes - 1) / kLanes;
    std::vector<uint32_t> scratch((size_t)ntiles * g.tile_scr_words);
    std::vector<float> vel((size_t)lds_rows(g) * kLanes);
    std::vector<float> ws((size_t)ntiles * art_ws_words(g.max_b) * kLanes);
    for (int w = 0; w < count; w++) {
        if (step_mask && !step_mask[w]) continue;
        float* lane_ws = ws.data() + (size_t)(w / kLanes) * art_ws_words(g.max_b) * kLanes + w % kLanes;
        step_world_art(lane_of(tiles, scratch.data(), vel.data(), g, w), lane_ws, dt, substeps);
    }
}

/* emu_step_art with the reduced-coordinate integrator (b3_art_step). */
void emu_art_step(uint32_t* tiles, int count, unsigned long long sig, float dt, int substeps,
        const unsigned char* step_mask) {
    Geometry g;
    size_t wb;
    if (!geometry_of(sig, &g, &wb)) return;
    int ntiles = (count + kLanes - 1) / kLanes;
    std::vector<uint32_t> scratch((size_t)ntiles * g.tile_scr_words);
    std::vector<float> vel((size_t)lds_rows(g) * kLanes);
    std::vector<float> ws((size_t)ntiles * art_ws_words(g.max_b) * kLanes);
    for (int w = 0; w < count; w++) {
        if (step_mask && !step_mask[w]) continue;
        float* lane_ws = ws.data() + (size_t)(w / kLanes) * art_ws_words(g.max_b) * kLanes + w % kLanes;
        step_world_art_reduced(lane_of(tiles, scratch.data(), vel.data(), g, w), lane_ws, dt, substeps);
    }
}

void emu_inputs(uint32_t* tiles, int count, unsigned long long sig, int scene, unsigned long long seed, int step,
        const unsigned char* step_mask) {
    Geometry g;
    size_t wb;
    if (!geometry_of(sig, &g, &wb)) return;
    for (int w = 0; w < count; w++) {
        if (step_mask && !step_mask[w]) continue;
        Lane L = lane_of(tiles, nullptr, nullptr, g, w);
        scene_inputs(L, scene, seed, w, step);
    }
}

}  // extern "C"

/* ---- atan2f: the engine's fd_atan2f against this host's libm ---- */
#include <thread>

extern "C" {

/* Host libm atan2f over arrays (the values the reference's CPU path gets). */
void emu_libm_atan2f(const float* y, const float* x, float* out, long n) {
    for (long i = 0; i < n; i++) out[i] = atan2f(y[i], x[i]);
}

/* The engine's fd_atan2f over arrays, built for the host. */
void emu_fd_atan2f(const float* y, const float* x, float* out, long n) {
    for (long i = 0; i < n; i++) out[i] = fd_atan2f(y[i], x[i]);
}

static uint64_t emu_mix(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
static float emu_f(uint32_t u) { return __builtin_bit_cast(float, u); }
static bool emu_same(float a, float b) {
    return __builtin_bit_cast(uint32_t, a) == __builtin_bit_cast(uint32_t, b) || (a != a && b != b);
}

/* Counts inputs where fd_atanf (mode 0: every float with bits in [lo, hi))
 * or fd_atan2f (mode 1: n pairs from the twist's domain, x in [0, 1] and
 * y in [-1, 1] with uniform bit patterns; mode 2: n pairs of arbitrary bit
 * patterns) differs from libm, on `threads` threads. */
unsigned long long emu_atan_mismatches(int mode, unsigned long long lo, unsigned long long hi,
        unsigned long long seed, int threads) {
    std::vector<unsigned long long> bad(threads, 0);
    std::vector<std::thread> pool;
    for (int t = 0; t < threads; t++) {
        pool.emplace_back([&, t]() {
            unsigned long long a = lo + (hi - lo) * t / threads, b = lo + (hi - lo) * (t + 1) / threads;
            for (unsigned long long i = a; i < b; i++) {
                if (mode == 0) {
                    float x = emu_f((uint32_t)i);
                    bad[t] += !emu_same(atanf(x), fd_atanf(x));
                    continue;
                }
                uint64_t r = emu_mix(i ^ (seed << 40));
                float x, y;
                if (mode == 1) {
                    x = emu_f((uint32_t)(r % 0x3f800001u));
                    y = emu_f((uint32_t)((r >> 32) % 0x3f800001u) | ((uint32_t)(r >> 31) & 1u) << 31);
                } else {
                    x = emu_f((uint32_t)r);
                    y = emu_f((uint32_t)(r >> 32));
                }
                bad[t] += !emu_same(atan2f(y, x), fd_atan2f(y, x));
            }
        });
    }
    unsigned long long total = 0;
    for (int t = 0; t < threads; t++) {
        pool[t].join();
        total += bad[t];
    }
    return total;
}

/* Counts the floats with bits in [lo, hi) (NaNs skipped: their payloads
 * are not part of the contract) where the engine's or_sinf or or_cosf
 * differ from libm's sinf or cosf, on `threads` threads; sin and cos
 * counts go to out[0] and out[1]. */
void emu_sincos_mismatches(unsigned long long lo, unsigned long long hi, int threads, unsigned long long* out) {
    std::vector<unsigned long long> bs(threads, 0), bc(threads, 0);
    std::vector<std::thread> pool;
    for (int t = 0; t < threads; t++) {
        pool.emplace_back([&, t]() {
            unsigned long long a = lo + (hi - lo) * t / threads, b = lo + (hi - lo) * (t + 1) / threads;
            for (unsigned long long i = a; i < b; i++) {
                float x = emu_f((uint32_t)i);
                if (x != x) continue;
                bs[t] += !emu_same(sinf(x), or_sinf(x));
                bc[t] += !emu_same(cosf(x), or_cosf(x));
            }
        });
    }
    out[0] = out[1] = 0;
    for (int t = 0; t < threads; t++) {
        pool[t].join();
        out[0] += bs[t];
        out[1] += bc[t];
    }
}

/* The engine's or_sinf and or_cosf over arrays, built for the host. */
void emu_or_sincosf(const float* x, float* s, float* c, long n) {
    for (long i = 0; i < n; i++) {
        s[i] = or_sinf(x[i]);
        c[i] = or_cosf(x[i]);
    }
}

/* libm's sinf and cosf over arrays. */
void emu_libm_sincosf(const float* x, float* s, float* c, long n) {
    for (long i = 0; i < n; i++) {
        s[i] = sinf(x[i]);
        c[i] = cosf(x[i]);
    }
}

}  // extern "C"
