/*
 * b3_engine.h - C ABI of the MI355X batched stepping engine.
 *
 * The reference exposes its GPU path as header-only functions over a
 * strided B3Batch of AoS worlds (b3_batch.cuh:12-99).  This library keeps
 * the same names and semantics, but the worlds live on the device inside an
 * engine handle, in a structure-of-arrays layout, so each entry point takes
 * a B3Engine* where the reference takes a B3Batch.  Scenes are still built
 * on the host with the reference's creation API (b3_setup.h) and handed
 * over once.
 *
 * Conventions (docs/API.md:58-63, b3_batch.cuh:19-99):
 *   - functions return hipSuccess or a hipError_t and never abort;
 *   - invalid arguments give hipErrorInvalidValue with no mutation and no
 *     launch; an empty batch or dt == 0 is a successful no-op;
 *   - the *_gpu functions enqueue on `stream` without allocating or
 *     synchronising; execution errors surface at the caller's
 *     synchronisation point;
 *   - masks are one byte per world in device memory, nonzero selects.
 *     NULL selects every world, except the reset mask of
 *     b3_batch_step_gpu, where NULL resets none;
 *   - b3_engine_create is the only call that allocates device memory
 *     (except b3_engine_set_options turning on B3_ENGINE_ART_CONTACTS),
 *     and b3_engine_destroy the only one that frees it.
 */
#ifndef PUFFYSICS_AMD_B3_ENGINE_H
#define PUFFYSICS_AMD_B3_ENGINE_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>

#include "b3_types.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct B3Engine B3Engine;

/* Create an engine on the current HIP device holding copies of the host
 * worlds viewed by `worlds` (a B3Batch exactly as b3_batch_valid accepts,
 * b3_batch.cuh:21-27), whose B3World capacities are `config_signature`
 * (B3_CONFIG_SIGNATURE of the caller's build, 01_config.inl:70-74).  The
 * worlds are checked for in-range counts and body/shape indices.  Blocks
 * until the upload is complete. */
hipError_t b3_engine_create(B3Engine** out, B3Batch worlds, unsigned long long config_signature);

/* Free everything the engine allocated.  NULL is a no-op. */
hipError_t b3_engine_destroy(B3Engine* engine);

/* Number of worlds, or -1 for NULL. */
int b3_engine_count(const B3Engine* engine);

/* Register `count` contiguous host B3World snapshots used by the reset
 * paths (b3_batch_restore's `initial`, b3_batch.cuh:50-60).  Blocks until
 * the copy is complete. */
hipError_t b3_engine_set_snapshots(B3Engine* engine, const void* initial);

/* Replace the device worlds with the host worlds of `worlds` (same count
 * and signature as at creation).  Blocks until complete. */
hipError_t b3_engine_upload(B3Engine* engine, B3Batch worlds);

/* Copy the device worlds out into the host worlds viewed by `worlds`.
 * Every field the step reads or writes is exact; contact points at or
 * beyond a contact's point_count and contact slots at or beyond
 * contact_count hold whatever the device last wrote there.  Blocks until
 * complete. */
hipError_t b3_engine_download(B3Engine* engine, B3Batch worlds);

/* Restore the worlds selected by `reset` from the registered snapshots
 * (b3_batch_restore_gpu, b3_batch.cuh:91-99).  Restores every persistent
 * field: header, bodies, shapes, joints and the snapshot's live contacts. */
hipError_t b3_batch_restore_gpu(B3Engine* engine, const unsigned char* reset, hipStream_t stream);

/* Masked restore then masked step, fused in one launch: equal to
 * b3_batch_restore(reset_mask) followed by b3_batch_step(step_mask)
 * (b3_batch.cuh:39-60).  step_mask NULL steps every world, reset_mask NULL
 * restores none.  dt must be finite and >= 0, substeps >= 1
 * (b3_batch_step_gpu, b3_batch.cuh:81-89). */
hipError_t b3_batch_step_gpu(B3Engine* engine, float dt, int substeps, const unsigned char* step_mask,
    const unsigned char* reset_mask, hipStream_t stream);

/* Accumulate per-body forces and torques, and apply linear impulses, from
 * dense device arrays laid out [world][body][xyz] over the engine's
 * body capacity (max_bodies of the signature).  Each selected world gets,
 * for every body b < body_count, in this order:
 *   force += force[w][b]                       (b3_apply_force, 09_step.inl:132-134)
 *   torque += torque[w][b]                     (b3_apply_torque, 09_step.inl:136-138)
 *   lin_vel += inv_mass * impulse[w][b] if the body is dynamic
 *                                              (b3_apply_linear_impulse, 09_step.inl:140-146)
 * Any of the three arrays may be NULL to skip that input; `mask` NULL
 * selects every world. */
hipError_t b3_batch_apply_gpu(B3Engine* engine, const float* force, const float* torque,
    const float* linear_impulse, const unsigned char* mask, hipStream_t stream);

/* Per-world B3StepStats (02_types.inl:336-346, b3_step_stats in
 * 04_world.inl:59-77) into a device array of `count` records. */
hipError_t b3_batch_stats_gpu(B3Engine* engine, B3StepStats* out, hipStream_t stream);

/* Device view of the live worlds for fused observation kernels: word k of
 * world w is ((uint32_t*)tiles)[((w / 64) * world_words + k) * 64 + w % 64],
 * where world_words = sizeof(B3World) / 4 of the engine's signature. */
hipError_t b3_engine_device_view(const B3Engine* engine, void** tiles, size_t* world_words);

/* Step options, a bit set (0 after b3_engine_create).  No counterpart in
 * the reference, whose contact structs double as solver scratch.
 *
 * B3_ENGINE_KEEP_SOLVER_FIELDS: also write the fields b3_prepare_one_contact
 * derives for every new contact (08_contacts.inl:234-291: inv_mass_a/b,
 * inv_i_a/b, softness, normal_mass, rel_vel, lever, center_a/b,
 * tangent_mass, twist_mass, rolling_mass) to the world's contact rows.  The
 * engine's solver keeps them in its own scratch and every step rewrites them
 * before use, so without the option they hold stale values in downloaded
 * worlds; every other field, and every body and joint, is the same either
 * way.  Set it to compare whole B3World structs with the reference. */
#define B3_ENGINE_KEEP_SOLVER_FIELDS 1u
/* B3_ENGINE_ART_CONTACTS: the step of the reference built with
 * B3_ART_CONTACTS=1 (01_config.inl:176-187).  In a world with revolute
 * joints and contacts whose joint tree builds (b3_art_bind, b3_art.cuh:
 * 488-490), the contact warm start and sweeps apply impulses through the
 * tree's Delassus operator (08_contacts.inl:194-232, 422-437); other
 * worlds step as usual.  The contacts' solver fields are then always
 * written back.  Turning it on allocates a workspace of
 * 4 * count * ((171 + 22) * max_bodies + 209) bytes (the one exception to
 * b3_engine_create being the only allocating call); it is freed by
 * b3_engine_destroy.  This mode costs far more per contact than the
 * default, as in the reference.  The force-law entry points return
 * hipErrorNotSupported while it is on. */
#define B3_ENGINE_ART_CONTACTS 2u
/* B3_ENGINE_ONE_WAVE_PER_TILE: no counterpart in the reference (a launch
 * choice).  A batch of at most one 64-world tile per CU normally runs with
 * eight waves per tile: they share the narrowphase (its pairs are
 * independent; four to seven waves collide, as many as have LDS rows for
 * their clip polygons), the contact sweeps and warm start (contacts on
 * disjoint dynamic bodies, level by level, keeping every body's updates in
 * contact order), the velocity and position updates, the joint geometry
 * and, when the joint rows fit in LDS, the joint passes (by joint levels),
 * while wave 0 does the rest; contact-bound worlds split each tile over
 * `parts` = 2 or 4 such workgroups when the CUs allow.  That allocates at
 * creation a staging buffer of 4 * tiles * parts * 64 * (1 + max(40 *
 * max_shapes * (max_shapes - 1) / 2, 2 * max_contacts)) bytes.  Worlds of at
 * most two shapes (one candidate pair) always step one wave per tile.  This
 * option launches one wave per tile as for larger batches.  Results are
 * identical either way. */
#define B3_ENGINE_ONE_WAVE_PER_TILE 4u
hipError_t b3_engine_set_options(B3Engine* engine, unsigned int options);

/* b3_art_step (09_step.inl:266-323), which the reference defines only in
 * its B3_ART_CONTACTS=1 build, over the masked batch: the reduced-
 * coordinate integrator.  A world whose joints are all passive revolutes
 * (no motor, spring, limit or fixed rotation) and whose bodies are neither
 * kinematic nor axis-locked moves its joint trees by articulated-body
 * dynamics and forward kinematics, solves loop-closing joints as 5x5
 * blocks and its contacts with four articulated sweeps per solve
 * (b3_art.cuh:990-1032, 1123-1279); any other world, or one without
 * joints, takes b3_batch_step_gpu's step with articulated contacts.
 * Masks, fused restore, validation and errors as b3_batch_step_gpu;
 * hipErrorNotSupported unless B3_ENGINE_ART_CONTACTS is on (the
 * workspace).  Results follow libm's sinf, cosf and atan2f (the joint
 * angles), which the device's differ from in the last place. */
hipError_t b3_batch_art_step_gpu(B3Engine* engine, float dt, int substeps, const unsigned char* step_mask,
    const unsigned char* reset_mask, hipStream_t stream);

/* The step without allocation.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory at all, such as code under
 * HIP graph capture, tight serving loops and harnesses that forbid
 * hipMalloc, and that hold their worlds in their own device memory.  The
 * engine's step needs per-step scratch, which b3_batch_step_gpu takes from
 * the engine (allocated by b3_engine_create) and this entry point from a
 * fixed device array of the library.
 *
 * Steps the device-resident B3World structs viewed by `worlds` (a B3Batch
 * over device memory of the current device, as b3_batch_valid accepts,
 * with data, stride and world_offset multiples of 4) whose capacities are
 * `config_signature`, in place: the worlds selected by `active` (device
 * bytes, nonzero selects, NULL selects all) that are structurally valid
 * (counts within the capacities, every body and shape index in range).  A
 * world that is not selected or not valid is left exactly as it is, and
 * the call still returns hipSuccess: a corrupt world is skipped, not
 * reported.  The results equal b3_batch_step_gpu's on an engine with
 * default options.  dt must be finite and >= 0, substeps >= 1; an empty
 * batch or dt == 0 is a no-op.  Errors, all before any launch:
 * hipErrorInvalidValue for invalid arguments or for `worlds` / `active`
 * outside device memory, hipErrorInvalidDevice for another device's
 * memory, hipErrorOutOfMemory when one 64-world tile of these worlds with
 * its scratch exceeds the array.  Enqueues on `stream`; calls no
 * allocating routine.
 *
 * Limit: the array holds 64 MiB, reserved on each device the library runs
 * on until the process ends.  A tile of 64 worlds needs
 *   64 * (sizeof(B3World) + scratch per world) + 64
 * bytes of it; the per-step scratch per world is about the size of the
 * world (34.3 KB beside a 37.3 KB world of 17 bodies, 17 shapes, 64
 * contacts and 4 joints).  A call runs its batch in chunks of as many
 * tiles as the array holds (14 tiles, 896 worlds, of the first kind), one
 * launch of each kernel per chunk, in order on the stream; a large batch
 * therefore runs at a fraction of b3_batch_step_gpu's rate.
 *
 * Calls share the array of their GPU.  Each call's stream waits for the
 * previous call's last kernel on that GPU (an event the library records
 * after every call), so calls from different streams or host threads take
 * turns.  A call made while its stream is being captured into a HIP graph
 * neither waits nor records: the caller must order the graph's launches
 * against other calls of this entry point on that GPU, or they race.  The
 * array keeps the last call's contents; nothing in it needs clearing
 * between calls. */
hipError_t b3_batch_step_worlds_gpu(B3Batch worlds, unsigned long long config_signature, float dt, int substeps,
    const unsigned char* active, hipStream_t stream);

/* ---- the CPU step ----
 * The reference's host b3_step (09_step.inl:262-264) and b3_batch_step
 * (b3_batch.cuh:39-48), capacity-agnostic: the caller passes its
 * B3_CONFIG_SIGNATURE.  b3_setup.h wraps them under the reference's names
 * (b3_step, b3_batch_step).  They run the engine's own step built for the
 * host, in place on host B3World structs (4-byte aligned), with results
 * bit-identical to the reference's CPU path, prepared contact fields
 * included.  No HIP call; safe to call from several threads on disjoint
 * worlds. */
void b3_host_step(void* world, unsigned long long config_signature, float dt, int substeps);
int b3_host_batch_step(B3Batch batch, unsigned long long config_signature, float dt, int substeps,
    const unsigned char* active);

/* ---- per-substep force laws ----
 * The reference's optional force hook B3_USER_FORCES (01_config.inl:189-198,
 * 09_step.inl:20-53) is a macro compiled into the step: once per substep,
 * before the velocity update, it may add to each body's applied force and
 * torque; that substep integrates the sums, and the applied values are
 * restored for the next substep.  This library compiles its law into the
 * step kernel the same way, behind its own entry point:
 * b3_batch_step_gpu (same masks, fused restore, validation and errors) with
 * the law in the hook. */

/* Plummer-softened gravity between the bodies of each world
 * (nbody_rigid.cuh:15-66; NbodyConfig, nbody.cuh:40-46).  For each pair
 * i < j of bodies with nonzero masses, at least one of them dynamic,
 *   r = c_j - c_i,  f = r * (gravity * m_i * m_j / (|r|^2 + softening^2)^1.5)
 * is added to a dynamic i and subtracted from a dynamic j, where c is the
 * body's current center (center + delta_pos, as the hook reads poses).
 * `masses` is NULL or a device array [world][body] over the engine's body
 * capacity of gravitational masses >= 0 (the world-major `masses` of
 * b3_nbody_step_kernel, nbody_rigid.cuh:110-119); NULL uses 1 / inv_mass
 * for dynamic bodies and 0 for the rest (b3_nbody_masses,
 * nbody_rigid.cuh:14-33).  The law needs gravity >= 0 and softening > 0
 * (nbody_cfg_ok, nbody.cuh:44-46), else hipErrorInvalidValue. */
typedef struct B3GravityLaw {
    float gravity;
    float softening;
} B3GravityLaw;
hipError_t b3_batch_step_gravity_gpu(B3Engine* engine, float dt, int substeps, const unsigned char* step_mask,
    const unsigned char* reset_mask, B3GravityLaw law, const float* masses, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif
