/*
 * b3_engine_internal.h - engine handle layout shared by the library's own
 * translation units (not installed).
 */
#ifndef PUFFYSICS_AMD_B3_ENGINE_INTERNAL_H
#define PUFFYSICS_AMD_B3_ENGINE_INTERNAL_H

#include "b3_engine.h"
#include "b3d_lane.h"

struct B3Engine {
    int device;
    int count;
    int tiles;
    unsigned long long sig;
    b3d::Geometry g;
    size_t world_bytes;
    size_t tile_words;
    uint32_t* live;
    uint32_t* snap;          /* count * world_bytes, AoS reset snapshots */
    uint32_t* scratch;
    unsigned char* staging;  /* count * world_bytes, AoS, for up/download */
    size_t lds_bytes;
    unsigned int options;    /* B3_ENGINE_* step options */
    float* art_ws;           /* articulated-contact workspace, allocated when that option is first set */
    uint32_t* pair_stage;    /* small batches: the tile's waves share the narrowphase (b3d::PairStage) */
    size_t stage_tile_words;
    size_t lds_shared_bytes; /* LDS of a workgroup of kTileWaves waves */
    bool shared_masks;       /* ... which also split the candidate search (b3d::shared_masks) */
    bool joint_lds;          /* ... and keep the joint rows in LDS (b3d::joint_rows_fit) */
    int tile_parts;          /* workgroups per tile of the shared step (1, 2 or 4), each with its own
                                scratch and stage */
    bool joint_impulses_lds; /* the one-wave step keeps the joint impulses in LDS (b3d::ji_fit) */
};

/* Waves per tile when the narrowphase is shared (two per SIMD: the shared
 * kernel's ~240 VGPRs allow it); the first kClipWaves of them have LDS clip
 * rows and collide, all of them share the rest of the step. */
constexpr int kTileWaves = 8;
static_assert(b3d::kClipWaves <= kTileWaves, "the colliding waves are among the tile's");

/* A CU's LDS.  The dynamic-LDS limit of a kernel is one setting shared by
 * every engine in the process, so the library raises it to this maximum
 * (b3i_lds_limit) instead of one engine's size, which an engine created
 * later with a smaller size would otherwise lower under an earlier one. */
constexpr size_t kCuLdsBytes = 160u * 1024u;
inline hipError_t b3i_lds_limit(const void* kernel) {
    return hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kCuLdsBytes);
}

/* Set-up of the force-law kernels on the current device (b3_forces.hip). */
hipError_t b3i_forces_init();
/* The articulated-contact step (b3_art.hip): its workspace, then launches. */
hipError_t b3i_art_init(B3Engine* e);
hipError_t b3i_step_art(B3Engine* e, float dt, int substeps, const unsigned char* step_mask,
    const unsigned char* reset_mask, hipStream_t stream);

/* The engine's device is the current one. */
inline hipError_t on_device(const B3Engine* e) {
    int dev = -1;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return err;
    return dev == e->device ? hipSuccess : hipErrorInvalidDevice;
}

namespace b3d {

/* Restore the resetting worlds of tile `tile` from the snapshots, which are
 * kept as plain B3World structs (AoS): one world at a time, the 64 lanes
 * read 64 consecutive snapshot words and write them to their rows of the
 * tile.  A world's copy is cut into chunks of kRestoreChunk words; this
 * wave copies chunk k of every resetting world when k % nslices == slice,
 * so nslices waves share a tile's restores.  Only the worlds of the lanes
 * set in `lanes` are restored. */
constexpr int kRestoreBatch = 8, kRestoreChunk = 64 * kRestoreBatch;
__device__ inline void restore_tile(uint32_t* live, const uint32_t* snap, const Geometry& g, int count,
        const unsigned char* reset, int tile, int slice, int nslices, uint64_t lanes = ~0ull) {
    int lane = (int)(threadIdx.x & 63u);
    int w = tile * 64 + lane;
    int want = w < count && ((lanes >> lane) & 1u) && reset[w] != 0;
    uint64_t bits = __ballot(want);
    uint32_t* lt = live + (size_t)tile * g.world_words * 64;
    while (bits) {
        int l = __builtin_ctzll(bits);
        bits &= bits - 1;
        const uint32_t* src = snap + (size_t)(tile * 64 + l) * g.world_words;
        int lo[3], hi[3];
        restore_ranges(g, (int)src[H_CONTACT_COUNT], lo, hi);
        int chunk = 0;
        for (int r = 0; r < 3; r++) {
            for (int c0 = lo[r]; c0 < hi[r]; c0 += kRestoreChunk, chunk++) {
                if (chunk % nslices != slice) continue;
                /* kRestoreBatch 256-byte snapshot reads in flight before
                 * their writes (the reads do not depend on the writes: the
                 * snapshots and the live tiles are separate allocations).
                 * A word already equal to the snapshot's is not written:
                 * each write is 4 bytes of a 256-byte row, which the memory
                 * merges by reading and writing the whole sector, and most
                 * of a world (shapes, body and joint constants) does not
                 * change in a step. */
                int k0 = c0 + lane;
                uint32_t v[kRestoreBatch], cur[kRestoreBatch];
#pragma unroll
                for (int i = 0; i < kRestoreBatch; i++)
                    if (k0 + 64 * i < hi[r]) {
                        v[i] = src[k0 + 64 * i];
                        cur[i] = lt[(size_t)(k0 + 64 * i) * 64 + l];
                    }
#pragma unroll
                for (int i = 0; i < kRestoreBatch; i++)
                    if (k0 + 64 * i < hi[r] && cur[i] != v[i]) lt[(size_t)(k0 + 64 * i) * 64 + l] = v[i];
            }
        }
    }
}

}  // namespace b3d

#endif
