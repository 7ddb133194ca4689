/*
 * CPU oracle for the Gated DeltaNet decode and prefill paths.
 *
 * TEST INFRASTRUCTURE ONLY. Results are compared against this library: tests, the
 * smoke check and the CPU-baseline leg of the benchmark load it. The product path (the HIP
 * library) never calls it, and nothing in the product falls back to it.
 *
 * It restates, token by token, the recurrence computed by the reference's
 * kernels:
 *   gdn_decode/solution/triton/kernel.py:120-131   (GVA head map, gates)
 *   gdn_decode/solution/triton/kernel.py:165-170   (decay, delta rule, readout)
 *   gdn_decode/solution/triton/kernel.py:216-218   (scale, output)
 *   gdn_prefill/solution/triton/kernel.py:87-89    (cu_seqlens ranges)
 *   gdn_prefill/solution/triton/kernel.py:281-302  (zero-filled output, state copy)
 * The exact recurrence is evaluated: the reference prefill's fp8 Q.S0 term and its
 * +-88 log-decay clamps (gdn_prefill/solution/triton/kernel.py:159,166,173-187) are
 * deviations of that kernel from the recurrence and are not reproduced.
 *
 * Two instantiations share one body (gdn_oracle_body.h):
 *   *_f64 : every quantity in IEEE double (the parity target)
 *   *_f32 : float arithmetic in the reference's order (rounding-noise yardstick)
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static inline float bf16_to_f32(uint16_t bits)
{
    uint32_t u = (uint32_t)bits << 16;
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

#define REAL double
#define SFX f64
#define EXP exp
#define LOG log
#include "gdn_oracle_body.h"
#undef REAL
#undef SFX
#undef EXP
#undef LOG

#define REAL float
#define SFX f32
#define EXP expf
#define LOG logf
#include "gdn_oracle_body.h"
#undef REAL
#undef SFX
#undef EXP
#undef LOG

int oracle_abi_version(void) { return 1; }
