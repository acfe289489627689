/*
 * ulp_envelope.c - TEST INFRASTRUCTURE ONLY: the oracle with every sinf,
 * cosf and atan2f result moved at random by one unit in the last place
 * (up, down, or kept, from a seeded generator).
 *
 * The device's sinf, cosf and atan2f are not glibc's; the two can differ in
 * the last place.  Where a result goes through them (joint twist angles,
 * the reduced integrator's forward kinematics), the spread of this
 * library's results over a few seeds, measured against the plain oracle,
 * is the envelope that a faithful implementation with another libm lands
 * in.  Tests compare the device's deviation from the oracle with it.
 */
#include <math.h>

static unsigned long long g_state = 1;

void oulp_seed(unsigned long long seed) { g_state = seed * 2654435761ull + 1ull; }

static float oulp_nudge(float x) {
    g_state = g_state * 6364136223846793005ull + 1442695040888963407ull;
    switch ((int)((g_state >> 33) % 3ull)) {
    case 0: return nextafterf(x, INFINITY);
    case 1: return nextafterf(x, -INFINITY);
    default: return x;
    }
}

float oulp_atan2f(float y, float x) { return oulp_nudge(atan2f(y, x)); }
float oulp_sinf(float x) { return oulp_nudge(sinf(x)); }
float oulp_cosf(float x) { return oulp_nudge(cosf(x)); }

#define atan2f oulp_atan2f
#define sinf oulp_sinf
#define cosf oulp_cosf
#include "b3cpu.c"
