/*
 * b3d_inputs.h - one world's per-step scene inputs, for one lane.
 *
 * The device twin of b3s_apply_inputs (puffysics_amd/scenes/b3_scenes.h):
 * the same counter-based draws and the same float operations in the same
 * order, applied to a world's transposed words.  The creation-side calls it
 * stands in for are b3_apply_force / b3_apply_torque /
 * b3_apply_linear_impulse (src/puffysics/09_step.inl:132-146) and
 * b3_joint_set_spring (src/puffysics/06_joints.inl:132-138).
 */
#ifndef PUFFYSICS_AMD_B3D_INPUTS_H
#define PUFFYSICS_AMD_B3D_INPUTS_H

#include "b3d_lane.h"
#include "../scenes/b3_scenes.h"

namespace b3d {

B3D_FN void scene_inputs(const Lane& L, int scene, unsigned long long seed, int w, int step) {
    const Geometry& g = L.g;
    int nb = body_count(L);
    if (scene == B3S_HOVER) {
        /* b3_apply_force(w, 1, (0, thrust, 0)) */
        if (nb > 1) st3(L.w, bw(L, 1, B_FORCE), add(ld3(L.w, bw(L, 1, B_FORCE)), v3(0.0f, b3s_hover_thrust(seed, w, step), 0.0f)));
    } else if (scene == B3S_STACK) {
        float imp[3];
        int b = b3s_stack_impulse(seed, w, step, imp);
        if (b >= 0 && b < nb && ldi(L.w, bw(L, b, B_TYPE)) == kDynamic)
            st3(L.w, bw(L, b, B_LIN_VEL), madd(ld3(L.w, bw(L, b, B_LIN_VEL)), ldf(L.w, bw(L, b, B_INV_MASS)),
                v3(imp[0], imp[1], imp[2])));
    } else if (scene == B3S_CHAIN) {
        if (b3s_chain_resample(step)) {
            int nj = clampi(ldi(L.w, H_JOINT_COUNT), 0, g.max_j);
            for (int j = 0; j < nj; j++) {
                /* b3_joint_set_spring(w, j, target, hertz, damping_ratio) */
                float hz = ldf(L.w, jw(L, j, J_HERTZ)), zeta = ldf(L.w, jw(L, j, J_DAMPING_RATIO));
                stf(L.w, jw(L, j, J_TARGET_ANGLE), clampf(b3s_chain_target(seed, w, step, j), -B3_PI, B3_PI));
                stf(L.w, jw(L, j, J_HERTZ), maxf(hz, 0.0f));
                stf(L.w, jw(L, j, J_DAMPING_RATIO), maxf(zeta, 0.0f));
            }
        }
    } else if (scene == B3S_ARM) {
        int nj = clampi(ldi(L.w, H_JOINT_COUNT), 0, g.max_j);
        for (int j = 0; j < nj; j++) {
            int a = ldi(L.w, jw(L, j, J_BODY_A)), b = ldi(L.w, jw(L, j, J_BODY_B));
            Q ra = ldq(L.w, bw(L, a, B_ROTATION)), lr = ldq(L.w, jw(L, j, J_LOCAL_ROT_A));
            float rot_a[4] = {ra.v.x, ra.v.y, ra.v.z, ra.s};
            float lrot[4] = {lr.v.x, lr.v.y, lr.v.z, lr.s};
            float tq[3];
            b3s_arm_torque(b3s_arm_action(seed, w, step, j), rot_a, lrot, tq);
            st3(L.w, bw(L, b, B_TORQUE), add(ld3(L.w, bw(L, b, B_TORQUE)), v3(tq[0], tq[1], tq[2])));
            if (ldi(L.w, bw(L, a, B_TYPE)) == kDynamic)
                st3(L.w, bw(L, a, B_TORQUE), add(ld3(L.w, bw(L, a, B_TORQUE)), v3(-tq[0], -tq[1], -tq[2])));
        }
    }
}

}  // namespace b3d

#endif
