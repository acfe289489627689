/*
 * flops.cpp - the oracle (b3cpu.c) re-compiled with an operation-counting
 * scalar, to count the algorithmic flops of the reference's b3_step.
 *
 * TEST INFRASTRUCTURE ONLY: it produces the committed per-configuration
 * flop counts (tests/golden/make_flops.py -> tests/golden/flops.json) that
 * the roofline's VALU fraction divides by; the engine never links it.
 *
 * b3cpu.c types every fp32 scalar of the step as `b3r`.  Here b3r is a
 * 4-byte class holding one float whose +, -, *, / (and their compound
 * assignments) each count one flop and round exactly as float arithmetic
 * does; sqrt counts one; negation, fabs, comparisons and copysign count
 * none.  The restatement has no fused multiply-add (the reference's
 * numerics forbid contraction), so nothing counts two.  One atan2f (the
 * hinge twist) counts 33: the adds, multiplies and divides of its main path
 * in the method glibc uses (one quotient, a 3-operation argument reduction,
 * the 11-term polynomial in 22 operations, 5 to recombine, 2 for the
 * quadrant).  The structs keep their layouts (static_asserts in b3cpu.c),
 * so the counting build steps the same B3World bytes, with the same
 * results bit for bit (tests/test_flops.py).
 */
#include <math.h>
#include <stdint.h>

namespace {
unsigned long long g_flops;
}

struct b3r {
    float v;
    b3r() = default;
    constexpr b3r(float x) : v(x) {}
    constexpr b3r(double x) : v((float)x) {}
    constexpr b3r(int x) : v((float)x) {}
    explicit operator float() const { return v; }
};
static_assert(sizeof(b3r) == sizeof(float), "b3r keeps the fp32 layout");

#define B3R_ARITH(op)                                                                         \
    static inline b3r operator op(b3r a, b3r b) { g_flops++; return b3r(a.v op b.v); }       \
    static inline b3r operator op(b3r a, float b) { g_flops++; return b3r(a.v op b); }       \
    static inline b3r operator op(float a, b3r b) { g_flops++; return b3r(a op b.v); }       \
    static inline b3r& operator op##=(b3r& a, b3r b) { g_flops++; a.v = a.v op b.v; return a; }
B3R_ARITH(+)
B3R_ARITH(-)
B3R_ARITH(*)
B3R_ARITH(/)
#undef B3R_ARITH
static inline b3r operator-(b3r a) { return b3r(-a.v); }
#define B3R_CMP(op)                                                                 \
    static inline bool operator op(b3r a, b3r b) { return a.v op b.v; }            \
    static inline bool operator op(b3r a, float b) { return a.v op b; }            \
    static inline bool operator op(float a, b3r b) { return a op b.v; }
B3R_CMP(<)
B3R_CMP(>)
B3R_CMP(<=)
B3R_CMP(>=)
B3R_CMP(==)
B3R_CMP(!=)
#undef B3R_CMP

#define B3R_TYPE 1
#define _Static_assert static_assert
static inline b3r o_sqrt(b3r x) { g_flops++; return b3r(sqrtf(x.v)); }
static inline b3r o_fabs(b3r x) { return b3r(fabsf(x.v)); }
static inline b3r o_atan2(b3r y, b3r x) { g_flops += 33; return b3r(atan2f(y.v, x.v)); }
static inline int o_isfinite(b3r x) { return isfinite(x.v); }
/* the force laws' and the reduced integrator's libm calls, uncounted (not
 * on the default step) */
static inline b3r cosf(b3r x) { return b3r(cosf(x.v)); }
static inline b3r sinf(b3r x) { return b3r(sinf(x.v)); }
static inline b3r powf(b3r x, b3r y) { return b3r(powf(x.v, y.v)); }
static inline b3r copysignf(b3r x, b3r y) { return b3r(copysignf(x.v, y.v)); }

extern "C" {
#include "b3cpu.c"

/* ocpu_batch_step (b3_batch.cuh:39-48) on the counting build; returns the
 * flops it took, or -1 when the arguments are invalid. */
long long ocount_batch_step(void* data, size_t stride, size_t world_offset, int count, unsigned long long sig,
        float dt, int substeps, const unsigned char* active) {
    unsigned long long before = g_flops;
    if (!ocpu_batch_step(data, stride, world_offset, count, sig, dt, substeps, active)) return -1;
    return (long long)(g_flops - before);
}
}
