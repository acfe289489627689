/*
 * b3_c99_step.c - a C99 caller of the library, built and run by
 * tests/test_host_step.py.  TEST INFRASTRUCTURE ONLY.
 *
 * Includes the public headers (b3_engine.h, b3_setup.h), builds a world
 * with the reference's creation API (a ground box, a hinged two-link arm
 * with a motor and limits, a sphere and a box), steps it with b3_step and
 * a batch of two copies with b3_batch_step, and writes the initial world
 * and both results as raw B3World bytes to the file named by argv[1].
 * Capacities: the library's capacity set 0 (16 bodies, 16 shapes, 32
 * contacts, 8 joints).
 */
#define B3_MAX_BODIES 16
#define B3_MAX_SHAPES 16
#define B3_MAX_CONTACTS 32
#define B3_MAX_JOINTS 8
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "b3_engine.h"
#include "b3_setup.h"

static int body(B3World* w, int type, float x, float y, float z) {
    B3BodyDef d = b3_default_body();
    d.type = type;
    d.position = b3_v(x, y, z);
    return b3_create_body(w, &d);
}

static void build(B3World* w) {
    B3ShapeDef sd = b3_default_shape();
    b3_world_init(w);
    int ground = body(w, B3_STATIC, 0.0f, -0.5f, 0.0f);
    b3_create_box(w, ground, b3_v(50.0f, 0.5f, 50.0f), &sd);
    int a = body(w, B3_DYNAMIC, 0.0f, 1.0f, 0.0f);
    b3_create_capsule(w, a, 0.3f, 0.1f, &sd);
    b3_finalize_mass(w, a);
    int b = body(w, B3_DYNAMIC, 0.0f, 1.8f, 0.0f);
    b3_create_capsule(w, b, 0.3f, 0.1f, &sd);
    b3_finalize_mass(w, b);
    int j0 = b3_create_revolute(w, ground, a, b3_v(0.0f, 1.1f, 0.0f), b3_v(0.0f, -0.4f, 0.0f),
        b3_v(0.0f, 0.0f, 1.0f));
    int j1 = b3_create_revolute(w, a, b, b3_v(0.0f, 0.4f, 0.0f), b3_v(0.0f, -0.4f, 0.0f), b3_v(0.0f, 0.0f, 1.0f));
    b3_joint_enable_motor(w, j0, 1);
    b3_joint_set_motor(w, j0, 0.5f, 5.0f);
    b3_joint_enable_limit(w, j1, 1);
    b3_joint_set_limits(w, j1, -0.5f, 0.5f);
    int s = body(w, B3_DYNAMIC, 0.7f, 0.4f, 0.1f);
    b3_create_sphere(w, s, b3_v(0.0f, 0.0f, 0.0f), 0.2f, &sd);
    b3_finalize_mass(w, s);
    int c = body(w, B3_DYNAMIC, -0.6f, 0.3f, 0.0f);
    b3_create_box(w, c, b3_v(0.2f, 0.2f, 0.2f), &sd);
    b3_finalize_mass(w, c);
}

int main(int argc, char** argv) {
    if (argc != 2) return 2;
    static B3World initial, single, pair[2];
    build(&initial);
    single = initial;
    for (int t = 0; t < 90; t++) {
        b3_apply_torque(&single, 1, b3_v(0.0f, 0.0f, t % 20 < 10 ? 2.0f : -2.0f));
        b3_step(&single, 1.0f / 60.0f, 4);
    }
    pair[0] = initial;
    pair[1] = initial;
    B3Batch batch = {pair, sizeof(B3World), 0, 2};
    unsigned char active[2] = {1, 0};
    for (int t = 0; t < 45; t++) {
        if (!b3_batch_step(batch, 1.0f / 60.0f, 4, t % 3 ? NULL : active)) return 3;
    }
    if (b3_batch_step(batch, 1.0f / 60.0f, 0, NULL) != 0) return 4;   /* substeps < 1: refused */
    FILE* f = fopen(argv[1], "wb");
    if (!f) return 5;
    fwrite(&initial, sizeof(B3World), 1, f);
    fwrite(&single, sizeof(B3World), 1, f);
    fwrite(pair, sizeof(B3World), 2, f);
    fclose(f);
    printf("sizeof(B3World) %zu signature %llx\n", sizeof(B3World), b3_config_signature());
    return 0;
}
