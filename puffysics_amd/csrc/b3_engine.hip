/*
 * b3_engine.hip - MI355X kernels and C ABI of the batched stepping engine.
 *
 * Launch geometry: every batch is split into tiles of 64 worlds, one
 * wave64 workgroup per tile, so each lane owns one world.  The grid is the
 * tile count (1024 workgroups at 65,536 worlds).  Worlds are stored as
 * word-transposed tiles (b3d_lane.h), which makes every per-field access of
 * a wave a single 256-byte row.
 *
 * Kernels:
 *   b3k_upload / b3k_download  AoS <-> tiles, transposed through LDS in
 *                              64 x 64 word blocks (both sides coalesced)
 *   b3k_step_select            b3_batch_step_worlds_gpu's worlds to step:
 *                              selected and structurally valid
 *   b3k_restore                masked restore from the snapshots (plain
 *                              B3World structs); four waves per tile, each
 *                              copying every fourth 512-word chunk of the
 *                              tile's resetting worlds with all 64 lanes
 *   b3k_step<JI, C0>           optional fused restore, then one b3_step per
 *                              selected lane; LDS holds the lane's clip
 *                              polygons, then its body velocities (JI: and
 *                              its joints' accumulated impulses; C0: contact
 *                              0's row kept for the step, for worlds of at
 *                              most two shapes)
 *   b3k_step_shared<Masks, JL> the same for batches of at most one tile per
 *                              CU, with the contact writes, preparation,
 *                              contact sweeps and body and joint work split
 *                              over eight waves per tile and the
 *                              narrowphase over the four to seven of them
 *                              that have LDS rows for clip polygons (Masks: the
 *                              candidate search too, for 12 shapes or more;
 *                              JL: the joint rows in LDS, when they fit)
 *   b3k_apply                  dense force / torque / impulse inputs
 *   b3k_stats                  per-world B3StepStats
 */
#include <hip/hip_runtime.h>

#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>

#include "b3_engine.h"
#include "b3_engine_internal.h"
#include "b3d_lane.h"

using namespace b3d;

namespace {

constexpr int kXposeThreads = 256;

/* ---- AoS <-> tile transposes ---- */

/* One workgroup per (tile, 64-word block): reads 64 worlds x 64 words with
 * each world's block contiguous, writes 64 rows of 64 lanes.  World w's
 * words start at aos[w * stride + offset] (stride, offset in words: a
 * B3Batch over device memory; world_words and 0 for packed worlds). */
__global__ __launch_bounds__(kXposeThreads) void b3k_upload(const uint32_t* __restrict__ aos,
        uint32_t* __restrict__ tiles, int count, int world_words, size_t stride, size_t offset) {
    __shared__ uint32_t blk[64][65];
    int tile = blockIdx.y;
    int k0 = blockIdx.x * 64;
    for (int e = threadIdx.x; e < 64 * 64; e += kXposeThreads) {
        int l = e >> 6, kk = e & 63;
        int w = tile * 64 + l;
        uint32_t v = 0;
        if (w < count && k0 + kk < world_words) v = aos[(size_t)w * stride + offset + k0 + kk];
        blk[l][kk] = v;
    }
    __syncthreads();
    size_t base = (size_t)tile * world_words * 64;
    for (int e = threadIdx.x; e < 64 * 64; e += kXposeThreads) {
        int kk = e >> 6, l = e & 63;
        if (k0 + kk < world_words) tiles[base + (size_t)(k0 + kk) * 64 + l] = blk[l][kk];
    }
}

__global__ __launch_bounds__(kXposeThreads) void b3k_download(const uint32_t* __restrict__ tiles,
        uint32_t* __restrict__ aos, int count, int world_words, size_t stride, size_t offset,
        const unsigned char* only) {
    __shared__ uint32_t blk[64][65];
    int tile = blockIdx.y;
    int k0 = blockIdx.x * 64;
    size_t base = (size_t)tile * world_words * 64;
    for (int e = threadIdx.x; e < 64 * 64; e += kXposeThreads) {
        int kk = e >> 6, l = e & 63;
        blk[l][kk] = k0 + kk < world_words ? tiles[base + (size_t)(k0 + kk) * 64 + l] : 0u;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < 64 * 64; e += kXposeThreads) {
        int l = e >> 6, kk = e & 63;
        int w = tile * 64 + l;
        if (w < count && k0 + kk < world_words && (!only || only[w]))
            aos[(size_t)w * stride + offset + k0 + kk] = blk[l][kk];
    }
}

/* kRestoreSlices waves per tile share its restores chunk by chunk: a tile
 * with several resetting worlds is then not one wave's long chain of
 * dependent rounds. */
constexpr int kRestoreSlices = 4;
__global__ __launch_bounds__(64) void b3k_restore(uint32_t* live, const uint32_t* snap, Geometry g, int count,
        const unsigned char* reset) {
    restore_tile(live, snap, g, count, reset, blockIdx.x / kRestoreSlices, blockIdx.x % kRestoreSlices,
        kRestoreSlices);
}

/* ---- the step ---- */

/* JI: the joints' accumulated impulses stay in LDS past the velocity rows
 * for the whole step (ji_fit; the launch gives ji_lds_rows words per lane),
 * instead of a read and a write of the joint's words in every solve.  C0:
 * contact 0's row is kept for the step (worlds of at most two shapes, whose
 * only contact it is), instead of a head and a row load in every sweep. */
template <bool JI, bool C0 = false>
__global__ __launch_bounds__(64) void b3k_step(uint32_t* live, const uint32_t* snap, uint32_t* scratch,
        Geometry g, int count, float dt, int substeps, const unsigned char* step_mask,
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
    Lane L = lane_view(live, scratch, vel_rows, g, tile, lane, opts);
    if (JI) L.ji = vel_rows + (size_t)ji_word(g) * kLanes + lane;
    step_world<false, false, JI, C0>(L, dt, substeps);
}

/* The step with the narrowphase and the contact sweeps shared by
 * kTileWaves waves per tile (small batches, whose one wave per tile would
 * leave most CUs idle): wave 0 steps its lanes' worlds as b3k_step does;
 * the other waves wait for its shape bounds (Masks: test their rows of the
 * bound pairs, then list their share of the candidates) or its candidate
 * lists, collide their share of the pairs into the stage (the first
 * clip_waves, which have clip rows), write their share of the new
 * contacts, prepare their share of them, then solve their share of each
 * level of every contact sweep and split the body and joint work.
 * Barriers: every thread of the workgroup reaches every __syncthreads.  A
 * tile with no stepping world returns as a whole (lane l of every wave
 * holds world 64 tile + l, so the ballot is the same in every wave).
 * Otherwise no thread returns: idle lanes (world past the batch or not in
 * the step mask) run the same control flow with L.active false, their
 * work skipped and their candidate and level counts zero; the barrier
 * count (find_pairs' fixed barriers, then 1 + nlev per levelled pass, with
 * nlev the tile's largest level count) is the same in every lane.
 * JL: the joint rows live in LDS past the level rows (joint_rows_fit). */
template <bool Masks, bool JL>
__global__ __launch_bounds__(64 * kTileWaves) void b3k_step_shared(uint32_t* live, const uint32_t* snap,
        uint32_t* scratch, uint32_t* stage, size_t stage_tile_words, Geometry g, int count, float dt, int substeps,
        const unsigned char* step_mask, const unsigned char* reset_mask, unsigned int opts, int parts) {
    extern __shared__ float lds[];
    int wave = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63u);
    /* `parts` workgroups share a tile: workgroup `group` steps the lanes
     * [part * 64 / parts, (part + 1) * 64 / parts) of tile group / parts,
     * with scratch and stage of its own (parts is 1, 2 or 4). */
    int group = blockIdx.x;
    int tile = group / parts, part = group % parts;
    int span = 64 / parts;
    uint64_t mine = (span == 64 ? ~0ull : ((1ull << span) - 1)) << (part * span);
    if (reset_mask) {
        restore_tile(live, snap, g, count, reset_mask, tile, wave, kTileWaves, mine);
        __syncthreads();
    }
    int w = tile * 64 + lane;
    bool stepping = w < count && ((mine >> lane) & 1u) && (!step_mask || step_mask[w]);
    if (!(dt > 0.0f) || __ballot(stepping) == 0) return;
    PairStage S;
    S.p = stage + (size_t)group * stage_tile_words + lane;
    S.cwaves = clip_waves(g, kTileWaves);
    S.clip = wave < S.cwaves ? lds + (size_t)clip_row_word(g, wave) * kLanes + lane : nullptr;
    S.wave = wave;
    S.waves = kTileWaves;
    S.lds_bounds = 1;
    Lane L = lane_view(live, scratch, lds, g, tile, lane, opts, group);
    L.st = S;
    L.staged = true;
    L.active = stepping;
    if (JL) L.jl = lds + (size_t)joint_lds_word(g) * kLanes + lane;
    if (wave == 0) {
        step_world<Masks, JL>(L, dt, substeps);
    } else {
        pair_helper<Masks>(L, S);
        sweep_helper<JL>(L, dt, substeps);
    }
}

/* ---- inputs and stats ---- */

__global__ __launch_bounds__(64) void b3k_apply(uint32_t* live, Geometry g, int count, const float* force,
        const float* torque, const float* impulse, const unsigned char* mask) {
    int tile = blockIdx.x;
    int lane = threadIdx.x;
    int w = tile * 64 + lane;
    if (w >= count || (mask && !mask[w])) return;
    Lane L;
    L.w = live + (size_t)tile * g.world_words * 64 + lane;
    L.g = g;
    int nb = body_count(L);
    for (int b = 0; b < nb; b++) {
        size_t in = ((size_t)w * g.max_b + b) * 3;
        if (force) {
            V3 f = v3(force[in], force[in + 1], force[in + 2]);
            st3(L.w, bw(L, b, B_FORCE), add(ld3(L.w, bw(L, b, B_FORCE)), f));
        }
        if (torque) {
            V3 t = v3(torque[in], torque[in + 1], torque[in + 2]);
            st3(L.w, bw(L, b, B_TORQUE), add(ld3(L.w, bw(L, b, B_TORQUE)), t));
        }
        if (impulse && ldi(L.w, bw(L, b, B_TYPE)) == kDynamic) {
            V3 p = v3(impulse[in], impulse[in + 1], impulse[in + 2]);
            st3(L.w, bw(L, b, B_LIN_VEL), madd(ld3(L.w, bw(L, b, B_LIN_VEL)), ldf(L.w, bw(L, b, B_INV_MASS)), p));
        }
    }
}

__global__ __launch_bounds__(64) void b3k_stats(const uint32_t* live, Geometry g, int count, B3StepStats* out) {
    int tile = blockIdx.x;
    int lane = threadIdx.x;
    int w = tile * 64 + lane;
    if (w >= count) return;
    const uint32_t* p = live + (size_t)tile * g.world_words * 64 + lane;
    B3StepStats s;
    s.body_count = ldi(p, H_BODY_COUNT);
    s.shape_count = ldi(p, H_SHAPE_COUNT);
    s.contact_count = ldi(p, H_CONTACT_COUNT);
    s.joint_count = ldi(p, H_JOINT_COUNT);
    s.body_overflow = ldi(p, B3D_W(B3WorldHeader, body_overflow));
    s.shape_overflow = ldi(p, B3D_W(B3WorldHeader, shape_overflow));
    s.joint_overflow = ldi(p, B3D_W(B3WorldHeader, joint_overflow));
    s.contact_overflow = ldi(p, H_CONTACT_OVERFLOW);
    s.contacts_dropped = ldi(p, H_CONTACTS_DROPPED);
    out[w] = s;
}

/* ---- host helpers ---- */

bool batch_valid(const B3Batch& b, size_t world_bytes) {
    if (b.count < 0) return false;
    if (b.count == 0) return true;
    return b.data != NULL && b.stride >= world_bytes && b.world_offset <= b.stride - world_bytes
        && (size_t)b.count <= SIZE_MAX / b.stride;
}

int host_word(const unsigned char* world, int k) {
    int v;
    memcpy(&v, world + (size_t)k * 4, 4);
    return v;
}

/* Structural checks that keep every index the kernels follow in range:
 * counts within the capacities, and every body and shape index a shape,
 * joint or contact holds below the world's counts.  `word(k)` reads word k
 * of the world. */
template <class Word>
B3D_FN bool world_ok(const Word& word, const Geometry& g) {
    int nb = word(H_BODY_COUNT), ns = word(H_SHAPE_COUNT);
    int nc = word(H_CONTACT_COUNT), nj = word(H_JOINT_COUNT);
    if (nb < 0 || nb > g.max_b || ns < 0 || ns > g.max_s || nc < 0 || nc > g.max_c || nj < 0 || nj > g.max_j)
        return false;
    for (int s = 0; s < ns; s++) {
        int b = word(g.so + s * kShapeWords + S_BODY);
        if (b < 0 || b >= nb) return false;
    }
    for (int j = 0; j < nj; j++) {
        int a = word(g.jo + j * kJointWords + J_BODY_A);
        int b = word(g.jo + j * kJointWords + J_BODY_B);
        if (a < 0 || a >= nb || b < 0 || b >= nb) return false;
    }
    for (int c = 0; c < nc; c++) {
        int base = g.co + c * kContactWords;
        int sa = word(base + C_SHAPE_A), sb = word(base + C_SHAPE_B);
        int ba = word(base + C_BODY_A), bb = word(base + C_BODY_B);
        int pc = word(base + C_POINT_COUNT);
        if (sa < 0 || sa >= ns || sb < 0 || sb >= ns || ba < 0 || ba >= nb || bb < 0 || bb >= nb || pc < 0
                || pc > kMaxManifold)
            return false;
    }
    return true;
}
bool world_valid(const unsigned char* wp, const Geometry& g) {
    return world_ok([wp](int k) { return host_word(wp, k); }, g);
}

/* The worlds b3_batch_step_worlds_gpu steps: selected by `active` (NULL:
 * all) and structurally valid (world_ok on the uploaded tile), so that a
 * corrupt caller world is left as it is rather than followed out of
 * range. */
__global__ __launch_bounds__(64) void b3k_step_select(const uint32_t* tiles, Geometry g, int count,
        const unsigned char* active, unsigned char* mask) {
    int tile = blockIdx.x;
    int lane = threadIdx.x;
    int w = tile * 64 + lane;
    if (w >= count) return;
    const uint32_t* p = tiles + (size_t)tile * g.world_words * 64 + lane;
    bool on = !active || active[w];
    mask[w] = on && world_ok([p](int k) { return ldi(p, k); }, g) ? 1 : 0;
}

/* Gather the batch's worlds into one contiguous host buffer. */
unsigned char* gather(const B3Batch& b, size_t world_bytes) {
    unsigned char* buf = (unsigned char*)malloc((size_t)b.count * world_bytes + 1);
    if (!buf) return NULL;
    for (int i = 0; i < b.count; i++)
        memcpy(buf + (size_t)i * world_bytes,
            (const unsigned char*)b.data + (size_t)i * b.stride + b.world_offset, world_bytes);
    return buf;
}

/* Host AoS buffer -> staging -> tiles (dst). */
hipError_t put_worlds(B3Engine* e, const unsigned char* host, uint32_t* dst) {
    if (e->count == 0) return hipSuccess;
    size_t bytes = (size_t)e->count * e->world_bytes;
    hipError_t err = hipMemcpy(e->staging, host, bytes, hipMemcpyHostToDevice);
    if (err != hipSuccess) return err;
    dim3 grid((unsigned)((e->g.world_words + 63) / 64), (unsigned)e->tiles);
    b3k_upload<<<grid, kXposeThreads>>>((const uint32_t*)e->staging, dst, e->count, e->g.world_words,
        (size_t)e->g.world_words, 0);
    err = hipGetLastError();
    if (err != hipSuccess) return err;
    return hipDeviceSynchronize();
}

/* ---- the step without allocation ----
 * b3_batch_step_worlds_gpu steps device-resident B3World structs in place
 * through the kernels of b3_batch_step_gpu, staging them as tiles in a
 * fixed device array instead of engine memory: a chunk's tiles
 * (world_words * 64 words each), then each tile's per-step scratch
 * (tile_scr_words), then one selection byte per world of the chunk.  A
 * batch larger than one chunk runs chunk after chunk on the caller's
 * stream.  Each GPU the library runs on holds its own copy of the array
 * from module load until the process ends. */
constexpr size_t kNoAllocWords = (size_t)16 << 20;            /* 64 MiB */
static __device__ __align__(256) uint32_t b3_noalloc_scratch[kNoAllocWords];

/* Per device, set up once with that device current: the array's device
 * address (the symbol's name in host code is a host-side stand-in, never a
 * device address: kernels get this pointer), and an event recorded after
 * each call's last kernel, which the next call's stream waits for, so that
 * calls on different streams or host threads take turns with the array. */
constexpr int kMaxDevices = 64;
struct NoAllocDevice {
    uint32_t* ptr;
    hipEvent_t last;
};
std::mutex g_noalloc_mu;
NoAllocDevice g_noalloc[kMaxDevices];

/* The current device's set-up; call with g_noalloc_mu held.  The event is
 * created by the first call that is not under graph capture (only those
 * use it). */
hipError_t noalloc_device(bool capturing, NoAllocDevice** out) {
    int dev = -1;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return err;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    NoAllocDevice& d = g_noalloc[dev];
    if (!d.ptr) {
        void* p = nullptr;
        if ((err = hipGetSymbolAddress(&p, HIP_SYMBOL(b3_noalloc_scratch))) != hipSuccess) return err;
        if (!p) return hipErrorInvalidSymbol;
        if ((err = b3i_lds_limit((const void*)b3k_step<false>)) != hipSuccess) return err;
        d.ptr = (uint32_t*)p;
    }
    if (!capturing && !d.last && (err = hipEventCreateWithFlags(&d.last, hipEventDisableTiming)) != hipSuccess)
        return err;
    *out = &d;
    return hipSuccess;
}

/* Words of the array per tile of geometry g: its worlds, their scratch and
 * their 64 selection bytes. */
size_t noalloc_tile_words(const Geometry& g) {
    return (size_t)g.world_words * 64 + (size_t)g.tile_scr_words + 64 / 4;
}

/* hipSuccess when the bytes [p, p + bytes) start and end in device memory
 * of the current device; hipErrorInvalidDevice when they are another
 * device's, hipErrorInvalidValue when they are not device memory.  A failed
 * lookup's error is cleared, so that it does not surface in a later call's
 * hipGetLastError. */
hipError_t device_range_here(const void* p, size_t bytes) {
    int dev = -1;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return err;
    const void* ends[2] = {p, (const unsigned char*)p + (bytes ? bytes - 1 : 0)};
    for (const void* q : ends) {
        hipPointerAttribute_t a;
        if (hipPointerGetAttributes(&a, q) != hipSuccess) {
            (void)hipGetLastError();
            return hipErrorInvalidValue;
        }
        if (a.type != hipMemoryTypeDevice && a.type != hipMemoryTypeManaged) return hipErrorInvalidValue;
        if (a.device != dev) return hipErrorInvalidDevice;
    }
    return hipSuccess;
}

}  // namespace

extern "C" {

hipError_t b3_engine_create(B3Engine** out, B3Batch worlds, unsigned long long config_signature) {
    if (!out) return hipErrorInvalidValue;
    *out = NULL;
    Geometry g;
    size_t world_bytes;
    if (!geometry_of(config_signature, &g, &world_bytes)) return hipErrorInvalidValue;
    if (!batch_valid(worlds, world_bytes)) return hipErrorInvalidValue;
    size_t lds = (size_t)lds_rows(g) * kLanes * sizeof(float);
    if (lds > kCuLdsBytes) return hipErrorInvalidValue;
    for (int i = 0; i < worlds.count; i++) {
        const unsigned char* wp = (const unsigned char*)worlds.data + (size_t)i * worlds.stride + worlds.world_offset;
        if (!world_valid(wp, g)) return hipErrorInvalidValue;
    }
    B3Engine* e = (B3Engine*)calloc(1, sizeof(B3Engine));
    if (!e) return hipErrorOutOfMemory;
    hipError_t err = hipGetDevice(&e->device);
    if (err != hipSuccess) {
        free(e);
        return err;
    }
    e->count = worlds.count;
    e->tiles = (worlds.count + 63) / 64;
    e->sig = config_signature;
    e->g = g;
    e->world_bytes = world_bytes;
    e->tile_words = (size_t)g.world_words * 64;
    /* the one-wave step keeps the joints' impulses in LDS when they fit */
    e->joint_impulses_lds = ji_fit(g);
    e->lds_bytes = e->joint_impulses_lds ? (size_t)ji_lds_rows(g) * kLanes * sizeof(float) : lds;
    err = b3i_lds_limit((const void*)b3k_step<false>);
    if (err == hipSuccess) err = b3i_lds_limit((const void*)b3k_step<true>);
    if (err == hipSuccess) err = b3i_lds_limit((const void*)b3k_step<false, true>);
    if (err == hipSuccess) err = b3i_lds_limit((const void*)b3k_step<true, true>);
    if (err == hipSuccess) err = b3i_lds_limit((const void*)b3k_step_shared<true, false>);
    if (err == hipSuccess) err = b3i_lds_limit((const void*)b3k_step_shared<false, false>);
    if (err == hipSuccess) err = b3i_lds_limit((const void*)b3k_step_shared<true, true>);
    if (err == hipSuccess) err = b3i_lds_limit((const void*)b3k_step_shared<false, true>);
    if (err != hipSuccess) {
        free(e);
        return err;
    }
    err = b3i_forces_init();
    if (err != hipSuccess) {
        free(e);
        return err;
    }
    if (e->tiles > 0) {
        size_t tiles_bytes = (size_t)e->tiles * e->tile_words * 4;
        if ((err = hipMalloc((void**)&e->live, tiles_bytes)) != hipSuccess
                || (err = hipMalloc((void**)&e->snap, (size_t)e->count * world_bytes)) != hipSuccess
                || (err = hipMalloc((void**)&e->staging, (size_t)e->count * world_bytes)) != hipSuccess) {
            (void)b3_engine_destroy(e);
            return err;
        }
        /* A batch of at most one tile per CU shares each tile's step among
         * kTileWaves waves (b3k_step_shared). */
        int cus = 0;
        /* wave 0's rows and the helpers' clip rows, then the old contact
         * keys, the overlap masks and the hit bits of the candidates */
        size_t shared_lds = (size_t)shared_lds_words(g) * kLanes * sizeof(float);
        /* wave 0's shape bounds stay in LDS until the overlap masks are
         * built (the helpers' clip rows are only used after them) */
        size_t bounds_lds = (size_t)(kClipWords + 6 * g.max_s) * kLanes * sizeof(float);
        if (bounds_lds > shared_lds) shared_lds = bounds_lds;
        /* and, past wave 0's rows, the contact levels of the shared sweeps,
         * then the joint rows when they fit */
        size_t sched_lds = (size_t)(lds_rows(g) + sched_words(g)) * kLanes * sizeof(float);
        if (sched_lds > shared_lds) shared_lds = sched_lds;
        bool joint_lds = joint_rows_fit(g);
        size_t joint_bytes = (size_t)(joint_lds_word(g) + joint_lds_words(g)) * kLanes * sizeof(float);
        if (joint_lds && joint_bytes > shared_lds) shared_lds = joint_bytes;
        if ((err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, e->device)) != hipSuccess) {
            (void)b3_engine_destroy(e);
            return err;
        }
        e->tile_parts = 1;
        /* Worlds of at most two shapes (one candidate pair, at most one
         * contact) leave the tile's waves nothing to share; their one-wave
         * step keeps that contact's row for the step (b3k_step<JI, true>):
         * the hover at 4,096 worlds 0.0398 ms shared, 0.0383 ms one-wave. */
        if (e->tiles <= cus && shared_lds <= kCuLdsBytes && g.max_s > 2) {
            size_t max_cand = (size_t)g.max_s * (size_t)(g.max_s - 1) / 2;
            size_t stage_words = max_cand * kStageWords;
            if ((size_t)stage_sched_words(g) > stage_words) stage_words = (size_t)stage_sched_words(g);
            e->stage_tile_words = (1 + stage_words) * kLanes;
            e->lds_shared_bytes = shared_lds;
            e->shared_masks = shared_masks(g);
            e->joint_lds = joint_lds;
            /* Contact-bound worlds step fewer than 64 to a workgroup when the
             * CUs allow: the narrowphase and the sweeps then take the union
             * of fewer worlds' code paths per step of their loops, on more
             * CUs.  Worlds of many shapes (whose candidate search uses the
             * overlap masks) step 16 to a workgroup, or 32; worlds with more
             * than four contacts per joint of capacity step 32.  Measured at
             * 4,096 worlds: the bin 0.842 ms (64) -> 0.724 (32) -> 0.700
             * (16); the stacks 0.228 -> 0.218 (32) -> 0.223 (16); the hover
             * (4 contacts, 2 joints) 0.040 -> 0.041 and the chains (32, 8)
             * 0.394 -> 0.397 -> 0.443, which stay at 64. */
            if (e->shared_masks && 4 * e->tiles <= cus) e->tile_parts = 4;
            else if (e->shared_masks && 2 * e->tiles <= cus) e->tile_parts = 2;
            else if (g.max_c > 4 * g.max_j && 2 * e->tiles <= cus) e->tile_parts = 2;
            err = hipMalloc((void**)&e->pair_stage,
                (size_t)e->tiles * e->tile_parts * e->stage_tile_words * sizeof(uint32_t));
            if (err != hipSuccess) {
                (void)b3_engine_destroy(e);
                return err;
            }
        }
        /* per-step scratch: one per workgroup of a tile */
        err = hipMalloc((void**)&e->scratch, (size_t)e->tiles * e->tile_parts * g.tile_scr_words * 4);
        if (err != hipSuccess) {
            (void)b3_engine_destroy(e);
            return err;
        }
        unsigned char* host = gather(worlds, world_bytes);
        if (!host) {
            (void)b3_engine_destroy(e);
            return hipErrorOutOfMemory;
        }
        /* Snapshots default to the initial worlds. */
        err = put_worlds(e, host, e->live);
        if (err == hipSuccess) err = hipMemcpy(e->snap, host, (size_t)e->count * world_bytes, hipMemcpyHostToDevice);
        free(host);
        if (err != hipSuccess) {
            (void)b3_engine_destroy(e);
            return err;
        }
    }
    *out = e;
    return hipSuccess;
}

hipError_t b3_engine_destroy(B3Engine* e) {
    if (!e) return hipSuccess;
    hipError_t first = hipSuccess;
    void* bufs[6] = {e->live, e->snap, e->scratch, e->staging, e->art_ws, e->pair_stage};
    for (void* p : bufs) {
        if (!p) continue;
        hipError_t err = hipFree(p);
        if (first == hipSuccess) first = err;
    }
    free(e);
    return first;
}

int b3_engine_count(const B3Engine* e) { return e ? e->count : -1; }

hipError_t b3_engine_set_snapshots(B3Engine* e, const void* initial) {
    if (!e || (e->count && !initial)) return hipErrorInvalidValue;
    hipError_t err = on_device(e);
    if (err != hipSuccess) return err;
    for (int i = 0; i < e->count; i++)
        if (!world_valid((const unsigned char*)initial + (size_t)i * e->world_bytes, e->g)) return hipErrorInvalidValue;
    if (e->count == 0) return hipSuccess;
    return hipMemcpy(e->snap, initial, (size_t)e->count * e->world_bytes, hipMemcpyHostToDevice);
}

hipError_t b3_engine_upload(B3Engine* e, B3Batch worlds) {
    if (!e || !batch_valid(worlds, e->world_bytes) || worlds.count != e->count) return hipErrorInvalidValue;
    hipError_t err = on_device(e);
    if (err != hipSuccess) return err;
    for (int i = 0; i < worlds.count; i++) {
        const unsigned char* wp = (const unsigned char*)worlds.data + (size_t)i * worlds.stride + worlds.world_offset;
        if (!world_valid(wp, e->g)) return hipErrorInvalidValue;
    }
    if (e->count == 0) return hipSuccess;
    unsigned char* host = gather(worlds, e->world_bytes);
    if (!host) return hipErrorOutOfMemory;
    err = put_worlds(e, host, e->live);
    free(host);
    return err;
}

hipError_t b3_engine_download(B3Engine* e, B3Batch worlds) {
    if (!e || !batch_valid(worlds, e->world_bytes) || worlds.count != e->count) return hipErrorInvalidValue;
    hipError_t err = on_device(e);
    if (err != hipSuccess) return err;
    if (e->count == 0) return hipSuccess;
    dim3 grid((unsigned)((e->g.world_words + 63) / 64), (unsigned)e->tiles);
    b3k_download<<<grid, kXposeThreads>>>(e->live, (uint32_t*)e->staging, e->count, e->g.world_words,
        (size_t)e->g.world_words, 0, nullptr);
    if ((err = hipGetLastError()) != hipSuccess) return err;
    unsigned char* host = (unsigned char*)malloc((size_t)e->count * e->world_bytes);
    if (!host) return hipErrorOutOfMemory;
    err = hipMemcpy(host, e->staging, (size_t)e->count * e->world_bytes, hipMemcpyDeviceToHost);
    if (err == hipSuccess) {
        for (int i = 0; i < e->count; i++)
            memcpy((unsigned char*)worlds.data + (size_t)i * worlds.stride + worlds.world_offset,
                host + (size_t)i * e->world_bytes, e->world_bytes);
    }
    free(host);
    return err;
}

hipError_t b3_batch_restore_gpu(B3Engine* e, const unsigned char* reset, hipStream_t stream) {
    if (!e) return hipErrorInvalidValue;
    if (e->count == 0) return hipSuccess;
    hipError_t err = on_device(e);
    if (err != hipSuccess) return err;
    if (!reset) {
        /* NULL restores every world: the whole structs, transposed into the tiles. */
        dim3 grid((unsigned)((e->g.world_words + 63) / 64), (unsigned)e->tiles);
        b3k_upload<<<grid, kXposeThreads, 0, stream>>>(e->snap, e->live, e->count, e->g.world_words,
            (size_t)e->g.world_words, 0);
        return hipGetLastError();
    }
    b3k_restore<<<e->tiles * kRestoreSlices, 64, 0, stream>>>(e->live, e->snap, e->g, e->count, reset);
    return hipGetLastError();
}

hipError_t b3_batch_step_gpu(B3Engine* e, float dt, int substeps, const unsigned char* step_mask,
        const unsigned char* reset_mask, hipStream_t stream) {
    if (!e || !isfinite(dt) || dt < 0.0f || substeps < 1) return hipErrorInvalidValue;
    if (e->count == 0) return hipSuccess;
    hipError_t err = on_device(e);
    if (err != hipSuccess) return err;
    if (dt == 0.0f) return reset_mask ? b3_batch_restore_gpu(e, reset_mask, stream) : hipSuccess;
    if (e->options & B3_ENGINE_ART_CONTACTS) return b3i_step_art(e, dt, substeps, step_mask, reset_mask, stream);
    if (e->pair_stage && !(e->options & B3_ENGINE_ONE_WAVE_PER_TILE)) {
        auto kernel = e->shared_masks ? (e->joint_lds ? b3k_step_shared<true, true> : b3k_step_shared<true, false>)
                                      : (e->joint_lds ? b3k_step_shared<false, true> : b3k_step_shared<false, false>);
        kernel<<<e->tiles * e->tile_parts, 64 * kTileWaves, e->lds_shared_bytes, stream>>>(e->live, e->snap,
            e->scratch, e->pair_stage, e->stage_tile_words, e->g, e->count, dt, substeps, step_mask, reset_mask,
            e->options, e->tile_parts);
        return hipGetLastError();
    }
    auto one_wave = e->g.max_s <= 2 ? (e->joint_impulses_lds ? b3k_step<true, true> : b3k_step<false, true>)
                                    : (e->joint_impulses_lds ? b3k_step<true> : b3k_step<false>);
    one_wave<<<e->tiles, 64, e->lds_bytes, stream>>>(e->live, e->snap, e->scratch, e->g, e->count, dt, substeps,
        step_mask, reset_mask, e->options);
    return hipGetLastError();
}

hipError_t b3_batch_apply_gpu(B3Engine* e, const float* force, const float* torque, const float* linear_impulse,
        const unsigned char* mask, hipStream_t stream) {
    if (!e) return hipErrorInvalidValue;
    if (e->count == 0 || (!force && !torque && !linear_impulse)) return hipSuccess;
    hipError_t err = on_device(e);
    if (err != hipSuccess) return err;
    b3k_apply<<<e->tiles, 64, 0, stream>>>(e->live, e->g, e->count, force, torque, linear_impulse, mask);
    return hipGetLastError();
}

hipError_t b3_batch_stats_gpu(B3Engine* e, B3StepStats* out, hipStream_t stream) {
    if (!e || (e->count && !out)) return hipErrorInvalidValue;
    if (e->count == 0) return hipSuccess;
    hipError_t err = on_device(e);
    if (err != hipSuccess) return err;
    b3k_stats<<<e->tiles, 64, 0, stream>>>(e->live, e->g, e->count, out);
    return hipGetLastError();
}

hipError_t b3_engine_device_view(const B3Engine* e, void** tiles, size_t* world_words) {
    if (!e || !tiles || !world_words) return hipErrorInvalidValue;
    *tiles = e->live;
    *world_words = (size_t)e->g.world_words;
    return hipSuccess;
}

hipError_t b3_engine_set_options(B3Engine* e, unsigned int options) {
    if (!e || (options & ~(B3_ENGINE_KEEP_SOLVER_FIELDS | B3_ENGINE_ART_CONTACTS | B3_ENGINE_ONE_WAVE_PER_TILE)))
        return hipErrorInvalidValue;
    if (options & B3_ENGINE_ART_CONTACTS) {
        hipError_t err = on_device(e);
        if (err == hipSuccess) err = b3i_art_init(e);
        if (err != hipSuccess) return err;
    }
    e->options = options;
    return hipSuccess;
}

hipError_t b3_batch_step_worlds_gpu(B3Batch worlds, unsigned long long config_signature, float dt, int substeps,
        const unsigned char* active, hipStream_t stream) {
    Geometry g;
    size_t world_bytes;
    if (!geometry_of(config_signature, &g, &world_bytes)) return hipErrorInvalidValue;
    if (!batch_valid(worlds, world_bytes) || !isfinite(dt) || dt < 0.0f || substeps < 1) return hipErrorInvalidValue;
    if (((uintptr_t)worlds.data | worlds.stride | worlds.world_offset) & 3u) return hipErrorInvalidValue;
    if (worlds.count == 0 || dt == 0.0f) return hipSuccess;
    size_t lds = (size_t)lds_rows(g) * kLanes * sizeof(float);
    if (lds > kCuLdsBytes) return hipErrorInvalidValue;
    size_t chunk_tiles = kNoAllocWords / noalloc_tile_words(g);
    if (chunk_tiles == 0) return hipErrorOutOfMemory;   /* one tile of these worlds exceeds the array */
    size_t span = (size_t)(worlds.count - 1) * worlds.stride + worlds.world_offset + world_bytes;
    hipError_t err = device_range_here(worlds.data, span);
    if (err == hipSuccess && active) err = device_range_here(active, (size_t)worlds.count);
    if (err != hipSuccess) return err;
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    if ((err = hipStreamIsCapturing(stream, &capture)) != hipSuccess) return err;
    bool capturing = capture != hipStreamCaptureStatusNone;

    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    NoAllocDevice* nd = nullptr;
    if ((err = noalloc_device(capturing, &nd)) != hipSuccess) return err;
    /* Take turns with the previous call on this GPU, whatever its stream.  A
     * call under capture cannot wait for work outside the graph: the caller
     * orders the graph's launches against other calls. */
    if (!capturing && (err = hipStreamWaitEvent(stream, nd->last, 0)) != hipSuccess) return err;
    int chunk = (int)(chunk_tiles * 64 < (size_t)worlds.count ? chunk_tiles * 64 : (size_t)worlds.count);
    uint32_t* aos = (uint32_t*)worlds.data;
    size_t stride = worlds.stride / 4, offset = worlds.world_offset / 4;
    for (int first = 0; first < worlds.count; first += chunk) {
        int n = worlds.count - first < chunk ? worlds.count - first : chunk;
        int tiles = (n + 63) / 64;
        uint32_t* tile_words = nd->ptr;
        uint32_t* step_scratch = tile_words + (size_t)tiles * g.world_words * 64;
        unsigned char* select = (unsigned char*)(step_scratch + (size_t)tiles * g.tile_scr_words);
        uint32_t* chunk_aos = aos + (size_t)first * stride;
        const unsigned char* chunk_active = active ? active + first : nullptr;
        dim3 grid((unsigned)((g.world_words + 63) / 64), (unsigned)tiles);
        b3k_upload<<<grid, kXposeThreads, 0, stream>>>(chunk_aos, tile_words, n, g.world_words, stride, offset);
        b3k_step_select<<<tiles, 64, 0, stream>>>(tile_words, g, n, chunk_active, select);
        b3k_step<false><<<tiles, 64, lds, stream>>>(tile_words, nullptr, step_scratch, g, n, dt, substeps, select,
            nullptr, 0u);
        /* only the stepped worlds are written back: the others are not touched */
        b3k_download<<<grid, kXposeThreads, 0, stream>>>(tile_words, chunk_aos, n, g.world_words, stride, offset,
            select);
        if ((err = hipGetLastError()) != hipSuccess) return err;
    }
    if (!capturing && (err = hipEventRecord(nd->last, stream)) != hipSuccess) return err;
    return hipSuccess;
}

}  // extern "C"
