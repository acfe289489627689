/*
 * b3cpu.h - CPU oracle for the batched rigid-body step.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the
 * reference's default b3_step path (src/puffysics/03_math.inl ..
 * 09_step.inl, b3_batch.cuh) used to check the MI355X engine and to time a
 * CPU baseline.  Only tests/, __graft_entry__.smoke() and bench.py's CPU
 * baseline leg may load it; the engine never calls it.
 *
 * Worlds are raw B3World bytes (include/b3_types.h layout) whose capacities
 * are given by a config signature, so one build serves every capacity set.
 */
#ifndef PUFFYSICS_AMD_ORACLE_B3CPU_H
#define PUFFYSICS_AMD_ORACLE_B3CPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* sizeof(B3World) for a signature, or 0 when the signature is invalid. */
size_t ocpu_world_size(unsigned long long sig);
/* b3_step on one world (09_step.inl:262-264). */
void ocpu_step(void* world, unsigned long long sig, float dt, int substeps);
/* b3_step with a force law in the B3_USER_FORCES hook (01_config.inl:
 * 189-198, 09_step.inl:20-53): Plummer-softened gravity between the
 * world's bodies (nbody_rigid.cuh:15-66) at their current centers.
 * `masses` is NULL (1 / inv_mass of dynamic bodies) or body_count floats. */
void ocpu_step_gravity(void* world, unsigned long long sig, float dt, int substeps, float gravity,
    float softening, const float* masses);
/* b3_step built with B3_ART_CONTACTS=1 (01_config.inl:176-187): in a world
 * with revolute joints the warm start and the contact sweeps use
 * articulated responses (b3_art.cuh; 08_contacts.inl:194-232, 422-437). */
void ocpu_step_art(void* world, unsigned long long sig, float dt, int substeps);
/* b3_art_step (09_step.inl:266-323): the reduced-coordinate integrator of
 * passive revolute trees with loop cuts; other worlds take ocpu_step_art. */
void ocpu_art_step(void* world, unsigned long long sig, float dt, int substeps);
/* b3_find_contacts alone (08_contacts.inl:64-173). */
void ocpu_find_contacts(void* world, unsigned long long sig);
/* b3_batch_step (b3_batch.cuh:39-48): 1 on success, 0 on invalid input. */
int ocpu_batch_step(void* data, size_t stride, size_t world_offset, int count,
    unsigned long long sig, float dt, int substeps, const unsigned char* active);
/* b3_batch_restore (b3_batch.cuh:53-60). */
int ocpu_batch_restore(void* data, size_t stride, size_t world_offset, int count,
    unsigned long long sig, const void* initial, const unsigned char* reset);
/* b3_apply_force / _torque / _linear_impulse (09_step.inl:132-146). */
void ocpu_apply_force(void* world, unsigned long long sig, int body, float x, float y, float z);
void ocpu_apply_torque(void* world, unsigned long long sig, int body, float x, float y, float z);
void ocpu_apply_linear_impulse(void* world, unsigned long long sig, int body, float x, float y, float z);

#ifdef __cplusplus
}
#endif
#endif
