/*
 * ref_art.c - the reference's own b3_step built with B3_ART_CONTACTS=1.
 *
 * TEST INFRASTRUCTURE ONLY.  Compiled by oracle/Makefile from the reference
 * sources in place (puffysics.cuh, which includes b3_art.cuh in this mode;
 * nothing is copied), once per capacity set, into oracle/_ref/.  The tests
 * check the oracle's articulated-contact step and its reduced-coordinate
 * integrator (b3_art_step) against it.
 */
#define B3_ART_CONTACTS 1
#include "puffysics.cuh"

unsigned long long refa_sig(void) { return b3_config_signature(); }
void refa_step(void* world, float dt, int substeps) { b3_step((B3World*)world, dt, substeps); }
void refa_art_step(void* world, float dt, int substeps) { b3_art_step((B3World*)world, dt, substeps); }
