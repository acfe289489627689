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
};

#endif
