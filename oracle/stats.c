/*
 * stats.c - per-world aggregates and body checksums of a batch of worlds.
 *
 * Test infrastructure, like the rest of oracle/: the full-size parity tests
 * take these of the oracle's worlds after every vector step, and the same
 * statistics of the engine's worlds on the device.  They restate
 * tests/b3test.py's stats_of_block and body_hash (the numpy definitions,
 * which tests/test_oracle_known.py holds this file to) in C, because numpy
 * takes about 0.3 s per step over 65,536 worlds.
 *
 * Per world, over the bodies whose type is dynamic:
 *   mean height  = mean of center.y
 *   mean energy  = mean of 0.5 m |v|^2 + 0.5 w_b . diag(1/inv_inertia) w_b
 *                  + m g center.y,  w_b = R^T w  (the body-frame rate)
 * and over every body slot (live or not), the checksum
 *   sum_k word_k * weight_k  in float64,  weight_k = (k 2654435761 + 12345)
 *   mod 1023 + 1,  NaN floats counted as 0x7fc00000,
 * which is exact (every partial sum is an integer below 2^53) and changes
 * when any single word changes.
 */
#include <stddef.h>
#include <stdint.h>
#include <string.h>

enum { BODY_WORDS = 50, W_ROT = 3, W_CENTER = 7, W_LIN_VEL = 13, W_ANG_VEL = 16, W_INV_MASS = 32,
       W_INV_INERTIA = 33, W_TYPE = 48 };
static const uint32_t kCanonNan = 0x7fc00000u;
static const double kGravity = 9.81;
#define kMaxBodies 256

static double fw(const uint32_t* b, int k) {
    float f;
    memcpy(&f, b + k, sizeof f);
    return (double)f;
}

static double recip_pos(double x) { return x > 0.0 ? 1.0 / x : 0.0; }

/* worlds: count structs of world_bytes each; bodies_word: word offset of
 * the bodies array; max_b: its capacity (at most 256).  Any output may be
 * NULL. */
void ostat_bodies(const void* worlds, int count, size_t world_bytes, int bodies_word, int max_b, double* height,
                  double* energy, double* checksum) {
    if (max_b < 0 || max_b > kMaxBodies) return;
    double weights[kMaxBodies * BODY_WORDS];
    for (long long k = 0; k < (long long)max_b * BODY_WORDS; k++)
        weights[k] = (double)((k * 2654435761LL + 12345) % 1023 + 1);
    for (int i = 0; i < count; i++) {
        const uint32_t* w = (const uint32_t*)((const char*)worlds + (size_t)i * world_bytes) + bodies_word;
        double hsum = 0.0, esum = 0.0, sum = 0.0;
        int n = 0;
        for (int b = 0; b < max_b; b++) {
            const uint32_t* q = w + b * BODY_WORDS;
            if (checksum) {
                const double* wt = weights + b * BODY_WORDS;
                for (int k = 0; k < BODY_WORDS; k++) {
                    uint32_t word = q[k];
                    /* a NaN: all exponent bits set and a nonzero fraction */
                    if ((word & 0x7fffffffu) > 0x7f800000u) word = kCanonNan;
                    sum += (double)word * wt[k];
                }
            }
            if ((int32_t)q[W_TYPE] != 2) continue;
            n++;
            double m = recip_pos(fw(q, W_INV_MASS));
            double vx = fw(q, W_LIN_VEL), vy = fw(q, W_LIN_VEL + 1), vz = fw(q, W_LIN_VEL + 2);
            double v2 = vx * vx + vy * vy + vz * vz;
            double nx = -fw(q, W_ROT), ny = -fw(q, W_ROT + 1), nz = -fw(q, W_ROT + 2), qs = fw(q, W_ROT + 3);
            double wx = fw(q, W_ANG_VEL), wy = fw(q, W_ANG_VEL + 1), wz = fw(q, W_ANG_VEL + 2);
            double tx = 2.0 * (ny * wz - nz * wy), ty = 2.0 * (nz * wx - nx * wz), tz = 2.0 * (nx * wy - ny * wx);
            double lx = wx + qs * tx + (ny * tz - nz * ty);
            double ly = wy + qs * ty + (nz * tx - nx * tz);
            double lz = wz + qs * tz + (nx * ty - ny * tx);
            double rot = recip_pos(fw(q, W_INV_INERTIA)) * lx * lx + recip_pos(fw(q, W_INV_INERTIA + 1)) * ly * ly
                         + recip_pos(fw(q, W_INV_INERTIA + 2)) * lz * lz;
            double y = fw(q, W_CENTER + 1);
            hsum += y;
            esum += 0.5 * m * v2 + 0.5 * rot + m * kGravity * y;
        }
        if (n < 1) n = 1;
        if (height) height[i] = hsum / n;
        if (energy) energy[i] = esum / n;
        if (checksum) checksum[i] = sum;
    }
}
