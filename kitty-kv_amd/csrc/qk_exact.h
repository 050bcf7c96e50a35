// Exact QK operand of the MFMA decode kernel (decode_mfma.hip).
#pragma once
#include <cstdint>

namespace kitty {

typedef unsigned qk_u32x4 __attribute__((ext_vector_type(4)));

// The QK A operand q[d] * s_k[d] (both fp16) is carried by two MFMA rows of
// its head: a = fp16(q s) on the first, the rounding residual fp16(q s - a)
// on the second, and the two output rows are added.  The residual is exact:
// the product of two fp16 numbers has at most 22 significant bits, so what
// rounding to 11 drops fits in 11 more (a residual under the fp16 normal
// range is off by less than 2^-25).  Lanes set in `lanes` (the second rows)
// replace a by the residual with v_pk_fma_f16 under that exec mask; the
// others keep a.  The trailing s_nop covers the wait states a DPP
// instruction needs after an EXEC write.
__device__ __forceinline__ void qk_residual(qk_u32x4 &a, const qk_u32x4 &q, const qk_u32x4 &s, uint64_t lanes)
{
    unsigned a0 = a[0], a1 = a[1], a2 = a[2], a3 = a[3];
    uint64_t saved;
    asm volatile("s_mov_b64 %0, exec\n\t"
                 "s_and_b64 exec, exec, %13\n\t"
                 "v_pk_fma_f16 %1, %5, %9, %1 neg_lo:[0,0,1] neg_hi:[0,0,1]\n\t"
                 "v_pk_fma_f16 %2, %6, %10, %2 neg_lo:[0,0,1] neg_hi:[0,0,1]\n\t"
                 "v_pk_fma_f16 %3, %7, %11, %3 neg_lo:[0,0,1] neg_hi:[0,0,1]\n\t"
                 "v_pk_fma_f16 %4, %8, %12, %4 neg_lo:[0,0,1] neg_hi:[0,0,1]\n\t"
                 "s_mov_b64 exec, %0\n\t"
                 "s_nop 4"
                 : "=&s"(saved), "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3)
                 : "v"(q[0]), "v"(q[1]), "v"(q[2]), "v"(q[3]), "v"(s[0]), "v"(s[1]), "v"(s[2]), "v"(s[3]),
                   "s"(lanes));
    a = qk_u32x4{a0, a1, a2, a3};
}

// Lanes holding the second (residual) row of a head in the QK A operand:
// row r of lane l is l & 15; GQA 4 uses rows 4h, 4h + 1, GQA 8 rows 2h, 2h + 1.
// GQA 16 has no spare row and runs a second MFMA chain for the residual.
template <int GQ>
constexpr uint64_t kResidualLanes = GQ == 4 ? 0x2222222222222222ull : (GQ == 8 ? 0xAAAAAAAAAAAAAAAAull : 0ull);

} // namespace kitty
