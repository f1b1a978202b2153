/*
 * tg_xchg.hpp -- epoch-tagged slot exchanges between the workgroups of a
 * persistent kernel (internal).
 *
 * A slot is 16 bytes {tag, v0, v1, v2} written and read as one vector
 * access, so its tag and values arrive together.  A writer publishes with
 * put_slot; readers poll with poll_slots until every slot they need carries
 * the expected tag.  Cross-XCD slots are stored and loaded with device-scope
 * coherence (sc1: the store writes through to memory, the load does not take
 * a stale line from the reader's L2); slots read only inside the writer's
 * XCD may be stored plainly (the line stays in that XCD's L2) and are still
 * loaded with sc1, which bypasses the CU's L1.  Every wait is bounded: a
 * wait that runs out raises an abort word that releases every other waiter.
 */
#ifndef TG_XCHG_HPP
#define TG_XCHG_HPP
#include "tg_device.hpp"

namespace tg {

constexpr int CPOL_PLAIN = 0, CPOL_SC1 = 16;
constexpr unsigned SPIN_LIMIT = 1u << 20;

template <int POL>
__device__ inline void put_slot(Buf sl, uint32_t slot, unsigned tag, float a, float b, float c) {
    u32x4 v;
    v.x = tag;
    v.y = __float_as_uint(a);
    v.z = __float_as_uint(b);
    v.w = __float_as_uint(c);
    __builtin_amdgcn_raw_buffer_store_b128(v, sl.r, (int)(slot * 16u), 0, POL);
}

/* Polls this communication lane's share of `total` slots (flat indices
 * cl, cl + CL, ...; slot(f) maps a flat index to a slot) until each carries
 * `tag`, handing every arrived slot to take(f, v).  All pending slots are
 * re-read as one batch per round.  Returns false if the wait timed out or
 * another workgroup aborted. */
template <int CL, int MAXP, class Slot, class Take>
__device__ inline bool poll_slots(Buf sl, int cl, int total, unsigned tag, unsigned *abort_flag, Slot slot, Take take,
                                  unsigned *rounds = nullptr) {
    uint32_t pending = 0;
#pragma unroll
    for (int i = 0; i < MAXP; i++)
        if (cl + CL * i < total) pending |= 1u << i;
    unsigned spins = 0;
    while (pending) {
        u32x4 v[MAXP];
#pragma unroll
        for (int i = 0; i < MAXP; i++)
            if (pending & (1u << i))
                v[i] = __builtin_amdgcn_raw_buffer_load_b128(sl.r, (int)(slot(cl + CL * i) * 16u), 0, CPOL_SC1);
#pragma unroll
        for (int i = 0; i < MAXP; i++)
            if ((pending & (1u << i)) && v[i].x == tag) {
                take(cl + CL * i, v[i]);
                pending &= ~(1u << i);
            }
        if (!pending) break;
        if ((++spins & 63) == 0 && __hip_atomic_load(abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
            return false;
        if (rounds) *rounds = spins;
        if (spins > SPIN_LIMIT) {
            __hip_atomic_store(abort_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return false;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    return true;
}


}  // namespace tg
#endif
