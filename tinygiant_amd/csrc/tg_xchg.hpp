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
    bool ok = true;
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
        if ((++spins & 63) == 0 && __hip_atomic_load(abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
            ok = false;
            break;
        }
        if (rounds) *rounds = spins;
        if (spins > SPIN_LIMIT) {
            __hip_atomic_store(abort_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ok = false;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    /* Every load the loop issued has returned (each round waits for its
     * own), but the compiler cannot prove it for the loads of rounds a lane
     * skipped, and would otherwise wait for them (vmcnt(0), which also waits
     * for every untracked copy issued later) before it reuses their
     * registers.  A wait it can see, on the one exit, ends that; it costs
     * nothing here. */
    __builtin_amdgcn_s_waitcnt(0x0F70);   /* vmcnt(0), expcnt and lgkmcnt unchanged */
    return ok;
}


/* ---- launch epochs (persistent kernels) ----
 *
 * Exchange tags are epoch + layer + 1; the epoch lives in word 1 of the
 * kernel's sync buffer (word 0 is the abort flag), so a launch needs no
 * per-launch argument and can be replayed from a graph.  Thread 0 of every
 * workgroup reads it before the workgroup's first barrier; thread 0 of
 * workgroup 0 advances it by 2 L when its workgroup leaves.  Workgroup 0
 * cannot leave before every workgroup has published its first layer, so
 * every workgroup has read the old value by then; the next launch on the
 * stream sees the new one. */
__device__ inline unsigned read_epoch(unsigned *sync) {
    return __hip_atomic_load(sync + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void advance_epoch(unsigned *sync, unsigned epoch, int L) {
    if (blockIdx.x == 0 && threadIdx.x == 0)
        __hip_atomic_store(sync + 1, epoch + 2u * (unsigned)L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* ---- weight streams into LDS (persistent kernels) ----
 *
 * One 1 KiB direct-to-LDS copy: lane l moves the 16 bytes at byte offset
 * voff (its own) of the buffer `desc` to LDS address lds + 16 l (lds is
 * wave-uniform).  Issued from inline assembly, so the compiler does not
 * track it: it would otherwise make LDS reads of other arrays wait for the
 * copies still in flight (it cannot tell the arrays apart), which is the
 * overlap these kernels need.  The waves that issue copies wait for them
 * themselves (wait_copies) before the barrier that opens the phase reading
 * them.  Vector-memory waits the compiler emits for its own loads stay
 * correct: the counter completes in order, so untracked operations only
 * make those waits stricter. */
__device__ inline u32x4 buf_desc(const void *p, uint32_t nbytes) {
    const uint64_t a = (uint64_t)(uintptr_t)p;
    u32x4 d;
    d.x = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
    d.y = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32)) & 0xFFFFu;
    d.z = (uint32_t)__builtin_amdgcn_readfirstlane((int)nbytes);
    d.w = 0x00020000u;
    return d;
}
__device__ inline uint32_t lds_addr(const void *p) {
    return (uint32_t)__builtin_amdgcn_readfirstlane(
        (int)(uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p);
}
/* M0 holds the copy's LDS address.  M0 is a reserved register the compiler
 * does not let inline assembly clobber; the kernels that use these copies
 * set M0 nowhere else (their generated code has no other M0 write).
 * The s_mov and s_nop 3 put 5 wait states before the load: a vector memory
 * instruction may read an SGPR (the descriptor) only 5 wait states after a
 * VALU instruction wrote it (v_readlane restoring a spilled SGPR, for one),
 * and the compiler pads its own loads for that but not inline assembly
 * (the M0 write needs 1). */
__device__ inline void copy_lanes(const u32x4 &desc, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 3\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(lds), "v"(voff), "s"(desc)
                 : "memory");
}
/* the 1 KiB at byte offset off: lane l copies bytes off + 16 l .. + 15 */
__device__ inline void copy_1k(const u32x4 &desc, uint32_t off, uint32_t lds, int lane) {
    copy_lanes(desc, off + 16u * (uint32_t)lane, lds);
}

/* A wait the compiler sees (the intrinsic, not inline assembly), so its
 * own bookkeeping of outstanding loads is cleared too: otherwise it keeps
 * loads of paths a wave never takes as pending and later waits for them,
 * with vmcnt(0), in the middle of a phase whose copies should stay in
 * flight.  It keeps such a wait as written. */
__device__ inline void wait_copies() {
    __builtin_amdgcn_s_waitcnt(0x0F70);   /* vmcnt(0); expcnt and lgkmcnt unchanged */
    asm volatile("" ::: "memory");
}
/* wait until at most N of the wave's vector memory operations are in flight */
template <int N>
__device__ inline void wait_copies_but() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

/* Workgroup barrier for the layer loops: waits for the wave's LDS accesses
 * (lgkmcnt) and meets the other waves; the memory clobber keeps the
 * compiler from moving accesses across it.  __syncthreads() (and a release
 * fence on LDS alone) would also wait for the wave's outstanding
 * direct-to-LDS copies (they count as vector memory operations), which must
 * stay in flight across the phases they overlap.  A wave whose copies a
 * phase reads waits for them itself (wait_copies) before the barrier that
 * opens that phase; nothing a workgroup stores to global memory inside a
 * layer is read back by that workgroup. */
__device__ inline void bar_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

}  // namespace tg
#endif
