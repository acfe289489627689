/*
 * b3d_forces.h - the built-in per-substep force law for the B3_USER_FORCES
 * hook (01_config.inl:189-198, 09_step.inl:20-53), run by
 * step_world(L, dt, substeps, law) of b3d_lane.h.  Host and device code,
 * like the lane code.
 */
#ifndef PUFFYSICS_AMD_B3D_FORCES_H
#define PUFFYSICS_AMD_B3D_FORCES_H

#include "b3d_lane.h"

namespace b3d {

/* Plummer-softened gravity between the bodies of one world
 * (nbody_rigid.cuh:15-66), as a force law: the sources sit at the current
 * centers (center + delta_pos), and the masses are the caller's
 * gravitational masses or, without them, 1 / inv_mass of the dynamic bodies
 * (0 for the rest, which then neither feel nor source gravity).  Pairs run
 * i < j in body order; each pair adds its force to a dynamic i and
 * subtracts it from a dynamic j, so body i's sum takes the pairs (k, i),
 * k < i, first and then (i, j), j > i, as the reference's loop does. */
struct GravityLaw {
    static constexpr bool kActive = true;
    float gravity;
    float softening;
    const float* masses;  /* this world's gravitational masses, or null */

    B3D_MFN float mass(const ForceView& v, int b) const {
        if (masses) return masses[b];
        float im = v.inv_mass(b);
        return v.type(b) == kDynamic && im > 0.0f ? 1.0f / im : 0.0f;
    }
    B3D_MFN void operator()(const ForceView& v) const {
        float eps2 = softening * softening;
        int nb = v.body_count();
        for (int i = 0; i < nb; i++) {
            float mi = mass(v, i);
            if (mi == 0.0f) continue;
            int ti = v.type(i);
            V3 ci = add(v.center(i), v.delta_pos(i));
            V3 fi = v.force(i);
            for (int j = i + 1; j < nb; j++) {
                float mj = mass(v, j);
                int tj = v.type(j);
                if (mj == 0.0f || (ti != kDynamic && tj != kDynamic)) continue;
                V3 r = sub(add(v.center(j), v.delta_pos(j)), ci);
                float q = dot(r, r) + eps2;
                float inv = 1.0f / sqrtf(q);
                V3 f = scale(r, gravity * mi * mj * inv * inv * inv);
                if (ti == kDynamic) fi = add(fi, f);
                if (tj == kDynamic) v.set_force(j, sub(v.force(j), f));
            }
            v.set_force(i, fi);
        }
    }
};

}  // namespace b3d

#endif
