/*
 * tg_api.hip -- the C ABI of libtinygiant_hip.so.
 *
 * The reference's ctypes loader (tinygiant/_lib.py:39-93) binds 21 symbols of
 * csrc/libtinygiant.c.  This file implements the hot-path ones on the GPU:
 *   tg_moe_forward_rows_v2, tg_moe_forward_rows, tg_moe_forward,
 *   tg_expert_forward, tg_expert_forward_mixed, tg_expert_forward_rows,
 *   tg_matmul, tg_matmul_q4k, tg_matmul_q6k, tg_row_bytes,
 *   tg_mlock (uploads the range to HBM), tg_set_threads, tg_get_threads,
 * and the device-resident tg_hip_* extensions (include/tinygiant_hip.h).
 * The out-of-scope symbols (attention, norms, f32/f16 matvecs, prefetch
 * hints, the full transformer layer) live in tg_host_ops.cpp.
 *
 * Calls are synchronous like the reference's: outputs are complete on
 * return.  All work runs on one non-blocking stream of the current device
 * under one process-wide mutex.  HIP runtime failures abort the process
 * with a message; invalid arguments are reported on stderr and through
 * tg_hip_last_error() and leave the outputs untouched.
 */
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <fcntl.h>
#include <unistd.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <thread>
#include <vector>

#include "tg_decode.h"
#include "tg_head.h"
#include "tg_attn.h"
#include "tg_route.h"
#include "tg_kernels.h"
#include "tg_synth.h"

#define TG_API extern "C" __attribute__((visibility("default")))

namespace tg {
/* tg_decode_mx.hip: the gpt-oss step's gate and up matrices in its
 * wave-segment layout (bytes of one rewritten matrix, and the rewrite) */
size_t decode_mx_seg_bytes();
hipError_t launch_mx_wave_segments(const void *src, void *dst, hipStream_t st);
}  // namespace tg

using namespace tg;

/* Fixed scratch of tg_hip_matmul_dev_noalloc: the q8 rows of its inputs.
 * Every GPU the library runs on holds one copy until the process ends; in
 * host code the name is only a handle, so the kernels get the device
 * address hipGetSymbolAddress returns for it at set-up (Ctx::scratch). */
constexpr size_t NOALLOC_SCRATCH_BYTES = 384 << 10;
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

namespace {

std::recursive_mutex g_mu;
char g_err[1024];
int g_threads = 1;

void hip_fail(hipError_t e, const char *what, const char *file, int line) {
    fprintf(stderr, "libtinygiant_hip: %s failed: %s (%s:%d)\n", what, hipGetErrorString(e), file, line);
    fflush(stderr);
    abort();
}
#define HIPCHECK(x)                                              \
    do {                                                         \
        hipError_t e_ = (x);                                     \
        if (e_ != hipSuccess) hip_fail(e_, #x, __FILE__, __LINE__); \
    } while (0)

void set_err(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    fprintf(stderr, "libtinygiant_hip: %s\n", g_err);
    fflush(stderr);
}

/* ---- device context ---- */
struct Ctx {
    bool ready = false;
    int dev = 0;
    hipStream_t st = nullptr;
    /* grow-only device arena for per-call scratch, pinned host staging */
    uint8_t *arena = nullptr;
    size_t arena_cap = 0;
    uint8_t *pin = nullptr;
    size_t pin_cap = 0;
    /* coherent (uncached on the device) pinned rows that kernels read and
     * write in place: the input and output rows of the host-pointer MoE call */
    uint8_t *io = nullptr;
    size_t io_cap = 0;
    /* row-tile tickets of the host call's fused MoE combine (zero between calls) */
    unsigned *tickets = nullptr;
    int tickets_cap = 0;
    /* device address of this GPU's copy of `scratch` (below) */
    uint8_t *scratch = nullptr;
};
Ctx g;

void ensure_init() {
    if (g.ready) return;
    HIPCHECK(hipGetDevice(&g.dev));
    HIPCHECK(hipStreamCreateWithFlags(&g.st, hipStreamNonBlocking));
    HIPCHECK(hipGetSymbolAddress((void **)&g.scratch, HIP_SYMBOL(scratch)));
    g.ready = true;
}

uint8_t *arena(size_t n) {
    if (n > g.arena_cap) {
        if (g.arena) {
            HIPCHECK(hipStreamSynchronize(g.st));
            HIPCHECK(hipFree(g.arena));
        }
        size_t cap = std::max(n, (size_t)64 << 20);
        HIPCHECK(hipMalloc(&g.arena, cap));
        g.arena_cap = cap;
    }
    return g.arena;
}

uint8_t *pinned(size_t n) {
    if (n > g.pin_cap) {
        if (g.pin) {
            HIPCHECK(hipStreamSynchronize(g.st));
            HIPCHECK(hipHostFree(g.pin));
        }
        size_t cap = std::max(n, (size_t)4 << 20);
        HIPCHECK(hipHostMalloc(&g.pin, cap, hipHostMallocDefault));
        g.pin_cap = cap;
    }
    return g.pin;
}

uint8_t *io_rows(size_t n) {
    if (n > g.io_cap) {
        if (g.io) {
            HIPCHECK(hipStreamSynchronize(g.st));
            HIPCHECK(hipHostFree(g.io));
        }
        size_t cap = std::max(n, (size_t)1 << 20);
        HIPCHECK(hipHostMalloc(&g.io, cap, hipHostMallocCoherent));
        g.io_cap = cap;
    }
    return g.io;
}

/* n zeroed ticket words on the device, queued on the library stream; every
 * kernel that takes tickets leaves them zero again */
unsigned *host_call_tickets(int n) {
    if (n > g.tickets_cap) {
        if (g.tickets) {
            HIPCHECK(hipStreamSynchronize(g.st));
            HIPCHECK(hipFree(g.tickets));
        }
        const int cap = std::max(n, 4096);
        HIPCHECK(hipMalloc(&g.tickets, (size_t)cap * 4));
        HIPCHECK(hipMemsetAsync(g.tickets, 0, (size_t)cap * 4, g.st));
        g.tickets_cap = cap;
    }
    return g.tickets;
}

/* Bump allocator over a byte range, 256-byte aligned pieces. */
struct Bump {
    size_t off = 0;
    size_t take(size_t n) {
        size_t o = off;
        off += (n + 255) & ~(size_t)255;
        return o;
    }
};

/* MXFP4 matrices of registered ranges already scanned for the scale byte
 * 255 (mx_any_e255 below): (device address, bytes) -> found */
static std::map<std::pair<uint64_t, uint64_t>, bool> g_e255_known;

/* ---- HBM residency registry (tg_mlock) ---- */
struct Region {
    size_t len;
    uint8_t *dev;
};
std::map<uintptr_t, Region> g_regs;

/* device copy of [p, p+n) if that range lies inside one registered region */
const void *lookup(const void *p, size_t n) {
    if (!p || g_regs.empty()) return nullptr;
    uintptr_t a = (uintptr_t)p;
    auto it = g_regs.upper_bound(a);
    if (it == g_regs.begin()) return nullptr;
    --it;
    if (a >= it->first && a + n <= it->first + it->second.len) return it->second.dev + (a - it->first);
    return nullptr;
}

int do_register(const void *addr, size_t len) {
    if (!addr || len == 0) return 0;
    ensure_init();
    if (lookup(addr, len)) return 0;
    uintptr_t a = (uintptr_t)addr;
    auto it = g_regs.find(a);
    if (it != g_regs.end()) {   /* same start, longer range: replace */
        HIPCHECK(hipStreamSynchronize(g.st));
        HIPCHECK(hipFree(it->second.dev));
        g_regs.erase(it);
        g_e255_known.clear();
    }
    uint8_t *dev = nullptr;
    hipError_t e = hipMalloc(&dev, len);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        set_err("tg_mlock: cannot allocate %zu bytes of HBM (%s)", len, hipGetErrorString(e));
        return -1;
    }
    HIPCHECK(hipMemcpy(dev, addr, len, hipMemcpyHostToDevice));
    g_regs[a] = Region{len, dev};
    return 0;
}

/* ---- per-call input resolution: registered range or staged copy ---- */
struct Stager {
    struct Item {
        const void *host;
        size_t n;
        size_t off;
    };
    std::vector<Item> items;
    Bump *bump;
    /* returns an arena offset (for staged data) or the device address */
    uintptr_t resolve(const void *host, size_t n, bool *staged) {
        const void *d = lookup(host, n);
        if (d) {
            *staged = false;
            return (uintptr_t)d;
        }
        *staged = true;
        size_t off = bump->take(n);
        items.push_back({host, n, off});
        return off;
    }
};

bool fmt_ok(int fmt) { return fmt == TG_FMT_Q4K || fmt == TG_FMT_F16 || fmt == TG_FMT_Q6K || fmt == TG_FMT_MXFP4 || fmt == TG_FMT_Q80; }

size_t q8_bytes(int nrows, int ncols) {
    size_t nb = TG_Q8_NB(ncols);
    return (size_t)nrows * nb * (256 + 4 + 32 + 64 + 4);
}

Q8Rows q8_view(uint8_t *base, int nrows, int ncols, const float *f) {
    Q8Rows q;
    const size_t nb = TG_Q8_NB(ncols);
    q.nb = (int)nb;
    q.qs = (int8_t *)base;
    q.d = (float *)(base + (size_t)nrows * nb * 256);
    q.s32 = (int32_t *)((uint8_t *)q.d + (size_t)nrows * nb * 4);
    q.s16 = (int32_t *)((uint8_t *)q.s32 + (size_t)nrows * nb * 32);
    q.sum = (int32_t *)((uint8_t *)q.s16 + (size_t)nrows * nb * 64);
    q.f = f;
    q.fstride = ncols;
    return q;
}

/* ---- MoE plan: device tables + scratch for one call shape ---- */
struct HostPlan {
    int n = 0, k = 0, P = 0, D = 0, I = 0, act = 0, gate_fmt = 0;
    std::vector<uint64_t> gate, up, down, gbias, ubias, dbias;
    std::vector<int> down_fmt, p_off, p_row, p_exp, r_off, r_pair;
    std::vector<float> p_w;
    bool has_gb = false, has_ub = false, has_db = false;
    std::vector<int> fmts_present;
};

/* ---- MXFP4 scale byte 255 ----
 * The reference reads the e8m0 byte 255 as 2^127; the block-scaled MFMA
 * phases cannot (k_mx_scan_e255), so a layer whose active MXFP4 matrices hold
 * such a block runs the v_dot4 phases.  Registered ranges are immutable
 * device copies: their result is kept (until the range is unregistered). */
static unsigned *g_e255_flags = nullptr;
static size_t g_e255_cap = 0;

/* the active experts' MXFP4 matrices of a host plan (device addresses) */
static std::vector<std::pair<uint64_t, uint64_t>> mx_matrices(const HostPlan &h, std::vector<int> *which = nullptr) {
    std::vector<std::pair<uint64_t, uint64_t>> m;
    const uint64_t gb = (uint64_t)h.I * row_bytes(TG_FMT_MXFP4, h.D), db = (uint64_t)h.D * row_bytes(TG_FMT_MXFP4, h.I);
    for (int e = 0; e < h.n; e++) {
        if (h.p_off[e + 1] == h.p_off[e]) continue;
        if (h.gate_fmt == TG_FMT_MXFP4) {
            m.push_back({h.gate[e], gb});
            m.push_back({h.up[e], gb});
            if (which) which->insert(which->end(), {3 * e, 3 * e + 1});
        }
        if (h.down_fmt[e] == TG_FMT_MXFP4) {
            m.push_back({h.down[e], db});
            if (which) which->push_back(3 * e + 2);
        }
    }
    return m;
}

static bool mx_any_e255(const std::vector<std::pair<uint64_t, uint64_t>> &mats, const std::vector<char> &keep) {
    std::vector<size_t> todo;
    for (size_t i = 0; i < mats.size(); i++) {
        if (keep[i]) {
            auto it = g_e255_known.find(mats[i]);
            if (it != g_e255_known.end()) {
                if (it->second) return true;
                continue;
            }
        }
        todo.push_back(i);
    }
    if (todo.empty()) return false;
    if (todo.size() > g_e255_cap) {
        if (g_e255_flags) {
            HIPCHECK(hipStreamSynchronize(g.st));
            HIPCHECK(hipFree(g_e255_flags));
        }
        g_e255_cap = std::max<size_t>(todo.size(), 64);
        HIPCHECK(hipMalloc(&g_e255_flags, g_e255_cap * 4));
    }
    HIPCHECK(hipMemsetAsync(g_e255_flags, 0, todo.size() * 4, g.st));
    for (size_t j = 0; j < todo.size(); j++)
        launch_mx_scan_e255((const uint8_t *)(uintptr_t)mats[todo[j]].first, mats[todo[j]].second, g_e255_flags + j,
                            g.st);
    HIPCHECK(hipGetLastError());
    std::vector<unsigned> f(todo.size());
    HIPCHECK(hipMemcpyAsync(f.data(), g_e255_flags, f.size() * 4, hipMemcpyDeviceToHost, g.st));
    HIPCHECK(hipStreamSynchronize(g.st));
    bool any = false;
    for (size_t j = 0; j < todo.size(); j++) {
        if (keep[todo[j]]) g_e255_known[mats[todo[j]]] = f[j] != 0;
        any = any || f[j] != 0;
    }
    return any;
}


bool validate_moe(int gate_fmt, const int *down_fmts, int n, int k, int D, int I, int act) {
    if (n < 0 || k < 0 || D <= 0 || I <= 0) {
        set_err("moe: bad sizes n=%d k=%d D=%d I=%d", n, k, D, I);
        return false;
    }
    if (D % 32 || I % 32) {
        set_err("moe: embed_dim (%d) and inter_dim (%d) must be multiples of 32", D, I);
        return false;
    }
    if (!fmt_ok(gate_fmt) || gate_fmt == TG_FMT_F16) {
        set_err("moe: unsupported gate/up format %d (F16 gate/up dereferences NULL in the reference)", gate_fmt);
        return false;
    }
    if (act != TG_ACT_SILU && act != TG_ACT_GPTOSS) {
        set_err("moe: unknown activation %d", act);
        return false;
    }
    for (int e = 0; e < n; e++)
        if (!fmt_ok(down_fmts[e])) {
            set_err("moe: unsupported down format %d for expert %d", down_fmts[e], e);
            return false;
        }
    if ((uint64_t)I * row_bytes(gate_fmt, D) >= (1ull << 32) || (uint64_t)D * row_bytes(TG_FMT_F16, I) >= (1ull << 32)) {
        set_err("moe: expert matrices must be under 4 GiB");
        return false;
    }
    return true;
}

/* pairs in the reference's gather order (csrc/libtinygiant.c:1411-1423) */
void build_pairs(HostPlan &h, const float *row_weights) {
    h.p_off.assign(h.n + 1, 0);
    h.p_row.clear();
    h.p_exp.clear();
    h.p_w.clear();
    std::vector<std::vector<int>> per_row(h.k);
    for (int e = 0; e < h.n; e++) {
        h.p_off[e] = (int)h.p_row.size();
        for (int r = 0; r < h.k; r++) {
            float w = row_weights[(size_t)e * h.k + r];
            if (w == 0.f) continue;
            per_row[r].push_back((int)h.p_row.size());
            h.p_row.push_back(r);
            h.p_exp.push_back(e);
            h.p_w.push_back(w);
        }
    }
    h.p_off[h.n] = (int)h.p_row.size();
    h.P = (int)h.p_row.size();
    h.r_off.assign(h.k + 1, 0);
    h.r_pair.clear();
    for (int r = 0; r < h.k; r++) {
        h.r_off[r] = (int)h.r_pair.size();
        for (int p : per_row[r]) h.r_pair.push_back(p);
    }
    h.r_off[h.k] = (int)h.r_pair.size();
    h.fmts_present.clear();
    for (int e = 0; e < h.n; e++)
        if (h.p_off[e + 1] > h.p_off[e] &&
            std::find(h.fmts_present.begin(), h.fmts_present.end(), h.down_fmt[e]) == h.fmts_present.end())
            h.fmts_present.push_back(h.down_fmt[e]);
}

/* Lays out tables + scratch in `base` (device) and the table image in `img`
 * (host); returns MoeArgs pointing into base. */
struct Layout {
    size_t tables, tables_len, xin, xq, hidden, hq, part, out, xp, hp, ctr, total;
};

/* compute units of the current device (workgroups of the persistent phases) */
static int cu_count() {
    static int n = 0;
    if (n == 0) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
            n = std::min(v, QA_RING_MAX_G);
        else
            n = 256;
    }
    return n;
}

/* row-tile tickets of the fused combine: at most one per 4 rows of D */
static int moe_ctr_words(int D) { return D / 4 + 16; }

Layout plan_layout(const HostPlan &h) {
    Layout L;
    Bump b;
    const int n = h.n, k = h.k, P = std::max(h.P, 1);
    L.tables = b.take(0);
    size_t t = 0;
    t += 6 * (size_t)n * 8;                 /* gate, up, down, gbias, ubias, dbias */
    t += (size_t)n * 4;                     /* down_fmt */
    t += (size_t)(n + 1) * 4 + (size_t)P * 4 * 4 + (size_t)(k + 1) * 4 + 8;   /* p_off, p_row, p_exp, p_w, r_off, r_pair */
    t += (size_t)4 * (n + 1) * 4 + 16;      /* active expert lists and their cost prefixes */
    t += (size_t)n * sizeof(ExpDesc) + 16;  /* active expert descriptors */
    if (qa_ring_shape(h.gate_fmt, h.D, h.I))  /* the persistent gate/up phase's items and ranges */
        t += 2 * (size_t)(h.I / 16) * (P / 16 + n + 1) * 4 + (size_t)RING_REC * (P / 16 + n + 1) * 4 +
             2 * (QA_RING_MAX_G + 1) * 4 + 64;
    if (qb_ring_shape(h.I, h.D))  /* the persistent down phase's */
        t += 2 * (size_t)(h.D / 32) * (P / 16 + n + 1) * 4 + (size_t)RING_REC * (P / 16 + n + 1) * 4 +
             2 * (QA_RING_MAX_G + 1) * 4 + 64;
    L.tables_len = t + 64;
    b.take(L.tables_len);
    L.xin = b.take((size_t)k * h.D * 4);
    L.xq = b.take(q8_bytes(std::max(k, 1), h.D));
    L.hidden = b.take((size_t)P * h.I * 4);
    L.hq = b.take(q8_bytes(P, h.I));
    L.part = b.take((size_t)P * h.D * 4);
    /* fp8 halves of the q8 rows for the MXFP4 MFMA phases (2 bytes a value) */
    const bool mx_down = std::find(h.down_fmt.begin(), h.down_fmt.end(), (int)TG_FMT_MXFP4) != h.down_fmt.end();
    L.xp = h.gate_fmt == TG_FMT_MXFP4 ? b.take((size_t)std::max(k, 1) * h.D * 2) : 0;
    L.hp = mx_down ? b.take((size_t)P * h.I * 2) : 0;
    L.out = b.take((size_t)k * h.D * 4);
    L.ctr = b.take((size_t)moe_ctr_words(h.D) * 4);
    L.total = b.off;
    return L;
}

/* serialises the tables into img (host, tables_len bytes) and returns the
 * MoeArgs for a device base address */
MoeArgs plan_args(const HostPlan &h, const Layout &L, uint8_t *dev, uint8_t *img) {
    const int n = h.n, k = h.k, P = std::max(h.P, 1);
    size_t o = 0;
    auto put = [&](const void *src, size_t bytes) {
        size_t at = o;
        if (bytes) memcpy(img + o, src, bytes);
        o += (bytes + 7) & ~(size_t)7;
        return dev + L.tables + at;
    };
    MoeArgs a;
    memset(&a, 0, sizeof a);
    a.gate = (const uint64_t *)put(h.gate.data(), (size_t)n * 8);
    a.up = (const uint64_t *)put(h.up.data(), (size_t)n * 8);
    a.down = (const uint64_t *)put(h.down.data(), (size_t)n * 8);
    const uint64_t *gb = (const uint64_t *)put(h.gbias.data(), (size_t)n * 8);
    const uint64_t *ub = (const uint64_t *)put(h.ubias.data(), (size_t)n * 8);
    const uint64_t *db = (const uint64_t *)put(h.dbias.data(), (size_t)n * 8);
    a.gbias = h.has_gb ? gb : nullptr;
    a.ubias = h.has_ub ? ub : nullptr;
    a.dbias = h.has_db ? db : nullptr;
    a.down_fmt = (const int *)put(h.down_fmt.data(), (size_t)n * 4);
    a.p_off = (const int *)put(h.p_off.data(), (size_t)(n + 1) * 4);
    a.p_row = (const int *)put(h.p_row.data(), (size_t)h.P * 4);
    a.p_exp = (const int *)put(h.p_exp.data(), (size_t)h.P * 4);
    a.p_w = (const float *)put(h.p_w.data(), (size_t)h.P * 4);
    a.r_off = (const int *)put(h.r_off.data(), (size_t)(k + 1) * 4);
    a.r_pair = (const int *)put(h.r_pair.data(), (size_t)h.P * 4);
    (void)P;
    a.xin = (const float *)(dev + L.xin);
    a.xq = q8_view(dev + L.xq, std::max(k, 1), h.D, a.xin);
    a.hidden = (float *)(dev + L.hidden);
    a.hq = q8_view(dev + L.hq, std::max(h.P, 1), h.I, a.hidden);
    a.part = (float *)(dev + L.part);
    a.xp = L.xp ? dev + L.xp : nullptr;
    a.hp = L.hp ? dev + L.hp : nullptr;
    a.out = (float *)(dev + L.out);
    a.ctr = (unsigned *)(dev + L.ctr);
    a.ctr_n = moe_ctr_words(h.D);
    a.n = n;
    a.k = k;
    a.P = h.P;
    a.D = h.D;
    a.I = h.I;
    a.act = h.act;
    a.gate_fmt = h.gate_fmt;
    a.gate_rb = row_bytes(h.gate_fmt, h.D);
    a.max_rows = 0;
    a.mx_aligned = 1;
    std::vector<int> act_a, act_b;
    for (int e = 0; e < n; e++) {
        if (h.p_off[e + 1] == h.p_off[e]) continue;
        a.max_rows = std::max(a.max_rows, h.p_off[e + 1] - h.p_off[e]);
        if (h.gate_fmt == TG_FMT_MXFP4 && ((h.gate[e] | h.up[e]) & 15)) a.mx_aligned = 0;
        if (h.down_fmt[e] == TG_FMT_MXFP4 && (h.down[e] & 15)) a.mx_aligned = 0;
        act_a.push_back(e);
        if (h.down_fmt[e] == TG_FMT_MXFP4) act_b.push_back(e);
    }
    a.n_act_a = (int)act_a.size();
    a.n_act_b = (int)act_b.size();
    /* cost of one item (16 rows of an expert) in the MFMA phases, in
     * quarter microseconds measured for D = I = 2880: one slab with its
     * first pass of 16 pairs (gate/up 10, down 5), and 19 / 18 per further
     * pass, which waits for its q8 operands */
    std::vector<int> cum;
    auto prefix = [&](const std::vector<int> &lst, int rows, int base, int per_pass) {
        int c = 0;
        cum.push_back(0);
        for (int e : lst) {
            const int passes = (h.p_off[e + 1] - h.p_off[e] + 15) / 16;
            c += ((rows + 15) / 16) * (base + per_pass * (passes - 1));
            cum.push_back(c);
        }
    };
    prefix(act_a, h.I, 10, 19);
    prefix(act_b, h.D, 5, 18);
    std::vector<ExpDesc> ed(a.n_act_a);
    for (int i = 0; i < a.n_act_a; i++) {
        const int e = act_a[i];
        ExpDesc &d = ed[i];
        memset(&d, 0, sizeof d);
        d.gate = h.gate[e];
        d.up = h.up[e];
        d.down = h.down[e];
        d.e = e;
        d.p0 = h.p_off[e];
        d.np = h.p_off[e + 1] - h.p_off[e];
        d.down_fmt = h.down_fmt[e];
        for (int s = 0; s < std::min(d.np, EXP_ROWS); s++) d.row[s] = h.p_row[d.p0 + s];
    }
    /* the busiest experts first: their workgroups (the most passes) start
     * first instead of trailing the launch */
    std::stable_sort(ed.begin(), ed.end(), [](const ExpDesc &x, const ExpDesc &y) { return x.np > y.np; });
    a.ed = (const ExpDesc *)put(ed.data(), ed.size() * sizeof(ExpDesc));
    if (qa_ring_shape(h.gate_fmt, h.D, h.I) && a.n_act_a > 0) {
        RingLists r;
        ring_items(ed.data(), a.n_act_a, h.I / 16, cu_count(), h.p_row.data(), P, r);
        a.rg_items = (const int *)put(r.items.data(), r.items.size() * 4);
        a.rg_rend = (const int *)put(r.rend.data(), r.rend.size() * 4);
        a.rg_runs = (const int *)put(r.runs.data(), r.runs.size() * 4);
        a.rg_run0 = (const int *)put(r.run0.data(), r.run0.size() * 4);
        a.rg_off = (const int *)put(r.off.data(), r.off.size() * 4);
        a.rg_n = (int)r.off.size() - 1;
    }
    if (qb_ring_shape(h.I, h.D) && a.n_act_a > 0) {
        RingLists r;
        ring_items(ed.data(), a.n_act_a, h.D / 32, cu_count(), h.p_row.data(), P, r);
        a.rb_items = (const int *)put(r.items.data(), r.items.size() * 4);
        a.rb_rend = (const int *)put(r.rend.data(), r.rend.size() * 4);
        a.rb_runs = (const int *)put(r.runs.data(), r.runs.size() * 4);
        a.rb_run0 = (const int *)put(r.run0.data(), r.run0.size() * 4);
        a.rb_off = (const int *)put(r.off.data(), r.off.size() * 4);
        a.rb_n = (int)r.off.size() - 1;
    }
    act_a.insert(act_a.end(), act_b.begin(), act_b.end());
    a.mx_act = (const int *)put(act_a.data(), act_a.size() * 4);
    a.mx_cum = (const int *)put(cum.data(), cum.size() * 4);
    return a;
}

/* The synchronous host-pointer MoE call behind every reference MoE symbol. */
/* q8 rows on the device -> the reference's 296-byte blocks on the host */
void q8_to_blocks(const Q8Rows &q, int nrows, void *out_blocks) {
    const size_t nq = (size_t)nrows * q.nb;
    std::vector<int8_t> qs(nq * 256);
    std::vector<float> d(nq);
    std::vector<int32_t> s32(nq * 8), sum(nq);
    HIPCHECK(hipMemcpyAsync(qs.data(), q.qs, qs.size(), hipMemcpyDeviceToHost, g.st));
    HIPCHECK(hipMemcpyAsync(d.data(), q.d, nq * 4, hipMemcpyDeviceToHost, g.st));
    HIPCHECK(hipMemcpyAsync(s32.data(), q.s32, nq * 32, hipMemcpyDeviceToHost, g.st));
    HIPCHECK(hipMemcpyAsync(sum.data(), q.sum, nq * 4, hipMemcpyDeviceToHost, g.st));
    HIPCHECK(hipStreamSynchronize(g.st));
    uint8_t *o = (uint8_t *)out_blocks;
    for (size_t i = 0; i < nq; i++) {
        uint8_t *blk = o + i * 296;
        memcpy(blk, &d[i], 4);
        memcpy(blk + 4, &sum[i], 4);
        memcpy(blk + 8, &s32[i * 8], 32);
        memcpy(blk + 40, &qs[i * 256], 256);
    }
}

void moe_host(const uint8_t *const *gate_ptrs, const uint8_t *const *up_ptrs, const void *const *down_ptrs,
              int gate_fmt, const int *down_fmts, const float *const *gate_bias, const float *const *up_bias,
              const float *const *down_bias, int act, int n, const float *row_weights, const float *inputs,
              float *output, int k, int D, int I, float *dbg_hidden = nullptr, void *dbg_hq = nullptr) {
    if (!validate_moe(gate_fmt, down_fmts, n, k, D, I, act)) return;
    if (n == 0 || k == 0) return;
    ensure_init();
    HostPlan h;
    h.n = n;
    h.k = k;
    h.D = D;
    h.I = I;
    h.act = act;
    h.gate_fmt = gate_fmt;
    h.down_fmt.assign(down_fmts, down_fmts + n);
    build_pairs(h, row_weights);
    if (h.P == 0) return;   /* every weight is zero: output unchanged */

    Layout L = plan_layout(h);
    Bump bump;
    bump.off = L.total;
    Stager sg;
    sg.bump = &bump;
    const size_t grb = (size_t)I * row_bytes(gate_fmt, D);
    std::vector<std::pair<uint64_t *, bool>> fix;   /* pointers that are arena offsets */
    h.gate.resize(n);
    h.up.resize(n);
    h.down.resize(n);
    h.gbias.assign(n, 0);
    h.ubias.assign(n, 0);
    h.dbias.assign(n, 0);
    h.has_gb = gate_bias != nullptr;
    h.has_ub = up_bias != nullptr;
    h.has_db = down_bias != nullptr;
    if (h.has_gb != h.has_ub) {
        set_err("moe: gate and up biases must both be given or both be NULL");
        return;
    }
    std::vector<char> staged_flags;
    struct Fix {
        std::vector<uint64_t> *vec;
        int idx;
    };
    std::vector<Fix> fixes;
    auto res = [&](std::vector<uint64_t> &vec, int e, const void *p, size_t bytes) {
        if (!p) {
            vec[e] = 0;
            return;
        }
        bool st;
        vec[e] = sg.resolve(p, bytes, &st);
        if (st) fixes.push_back({&vec, e});
    };
    for (int e = 0; e < n; e++) {
        if (h.p_off[e + 1] == h.p_off[e]) {   /* inactive expert: never read */
            h.gate[e] = h.up[e] = h.down[e] = 0;
            continue;
        }
        res(h.gate, e, gate_ptrs[e], grb);
        res(h.up, e, up_ptrs[e], grb);
        res(h.down, e, down_ptrs[e], (size_t)D * row_bytes(down_fmts[e], I));
        if (h.has_gb) res(h.gbias, e, gate_bias[e], (size_t)I * 4);
        if (h.has_ub) res(h.ubias, e, up_bias[e], (size_t)I * 4);
        if (h.has_db) res(h.dbias, e, down_bias[e], (size_t)D * 4);
    }
    uint8_t *dev = arena(bump.off);
    for (auto &f : fixes) (*f.vec)[f.idx] += (uint64_t)(uintptr_t)dev;

    /* the tables go over in one copy; the input rows are read and the output
     * rows accumulated in place in coherent pinned memory (the q8 kernel and
     * the combine reach them over the host link), which saves three copy
     * launches per call */
    const size_t io_len = (size_t)k * D * 4;
    uint8_t *img = pinned(L.tables_len);
    uint8_t *io = io_rows(2 * io_len);
    MoeArgs a = plan_args(h, L, dev, img);
    memcpy(io, inputs, io_len);
    memcpy(io + io_len, output, io_len);
    a.xin = (const float *)io;
    a.xq.f = a.xin;
    a.xin_remote = 1;
    a.out = (float *)(io + io_len);
    /* the arena is laid out afresh each call: the tickets live in a buffer
     * of their own that every fused combine leaves zeroed */
    a.ctr = host_call_tickets(moe_ctr_words(D));
    a.ctr_n = a.ctr ? moe_ctr_words(D) : 0;
    HIPCHECK(hipMemcpyAsync(dev + L.tables, img, L.tables_len, hipMemcpyHostToDevice, g.st));
    for (auto &it : sg.items) HIPCHECK(hipMemcpyAsync(dev + it.off, it.host, it.n, hipMemcpyHostToDevice, g.st));
    if (grouped_min_rows() > 0 && a.max_rows >= grouped_min_rows()) {
        /* the MFMA phases are a candidate: no e8m0 byte of 255 may reach
         * them (registered matrices are scanned once, staged ones per call) */
        std::vector<int> which;
        const auto mats = mx_matrices(h, &which);
        std::vector<char> keep(mats.size(), 1);
        for (auto &f : fixes) {
            const int part = f.vec == &h.gate ? 0 : f.vec == &h.up ? 1 : f.vec == &h.down ? 2 : -1;
            for (size_t i = 0; i < which.size(); i++)
                if (part >= 0 && which[i] == 3 * f.idx + part) keep[i] = 0;
        }
        a.mx_e255 = mx_any_e255(mats, keep) ? 1 : 0;
    }
    launch_moe(a, h.fmts_present.data(), (int)h.fmts_present.size(), g.st);
    HIPCHECK(hipGetLastError());
    HIPCHECK(hipStreamSynchronize(g.st));
    memcpy(output, io + io_len, io_len);
    if (dbg_hidden)
        HIPCHECK(hipMemcpy(dbg_hidden, a.hidden, (size_t)h.P * I * 4, hipMemcpyDeviceToHost));
    if (dbg_hq) q8_to_blocks(a.hq, h.P, dbg_hq);
}

void matmul_host(int fmt, const void *mat, const float *bias, const float *input, float *output, int nrows,
                 int ncols) {
    if (!fmt_ok(fmt)) {
        set_err("tg_matmul: unknown format %d", fmt);
        return;
    }
    if (ncols <= 0 || ncols % 32 || nrows < 0) {
        set_err("tg_matmul: ncols (%d) must be a positive multiple of 32", ncols);
        return;
    }
    if (nrows == 0) return;
    ensure_init();
    const size_t rb = row_bytes(fmt, ncols);
    Bump b;
    const size_t o_in = b.take((size_t)ncols * 4);
    const size_t o_q = b.take(q8_bytes(1, ncols));
    const size_t o_out = b.take((size_t)nrows * 4);
    Stager sg;
    sg.bump = &b;
    bool st_m = false, st_b = false;
    uintptr_t m = sg.resolve(mat, (size_t)nrows * rb, &st_m);
    uintptr_t bi = bias ? sg.resolve(bias, (size_t)nrows * 4, &st_b) : 0;
    uint8_t *dev = arena(b.off);
    if (st_m) m += (uintptr_t)dev;
    if (bias && st_b) bi += (uintptr_t)dev;
    HIPCHECK(hipMemcpyAsync(dev + o_in, input, (size_t)ncols * 4, hipMemcpyHostToDevice, g.st));
    for (auto &it : sg.items) HIPCHECK(hipMemcpyAsync(dev + it.off, it.host, it.n, hipMemcpyHostToDevice, g.st));
    Q8Rows q = q8_view(dev + o_q, 1, ncols, (const float *)(dev + o_in));
    if (fmt != TG_FMT_F16) launch_quantize((const float *)(dev + o_in), ncols, 1, ncols, q, g.st);
    launch_gemv(fmt, (const uint8_t *)m, nrows, ncols, (const float *)bi, q, 1, (float *)(dev + o_out), nrows, g.st);
    HIPCHECK(hipGetLastError());
    HIPCHECK(hipMemcpyAsync(output, dev + o_out, (size_t)nrows * 4, hipMemcpyDeviceToHost, g.st));
    HIPCHECK(hipStreamSynchronize(g.st));
}

}  // namespace

/* ===================== reference ABI (tinygiant/_lib.py) ===================== */

TG_API void tg_moe_forward_rows_v2(const uint8_t *const *gate_ptrs, const uint8_t *const *up_ptrs,
                                   const void *const *down_ptrs, int gate_fmt, const int *down_fmts,
                                   const float *const *gate_bias, const float *const *up_bias,
                                   const float *const *down_bias, int act, int n_experts, const float *row_weights,
                                   const float *inputs, float *output, int k, int embed_dim, int inter_dim) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    moe_host(gate_ptrs, up_ptrs, down_ptrs, gate_fmt, down_fmts, gate_bias, up_bias, down_bias, act, n_experts,
             row_weights, inputs, output, k, embed_dim, inter_dim);
}

/* tg_moe_forward_rows_v2 that also returns the stage outputs: the hidden
 * rows [pairs][inter_dim] (f32, pairs expert-major in gather order) and their
 * q8 quantization as 296-byte blocks [pairs][ceil(inter_dim/256)]. */
TG_API void tg_hip_moe_forward_stages(const uint8_t *const *gate_ptrs, const uint8_t *const *up_ptrs,
                                      const void *const *down_ptrs, int gate_fmt, const int *down_fmts,
                                      const float *const *gate_bias, const float *const *up_bias,
                                      const float *const *down_bias, int act, int n_experts,
                                      const float *row_weights, const float *inputs, float *output, int k,
                                      int embed_dim, int inter_dim, float *hidden_out, void *hq_blocks_out) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    moe_host(gate_ptrs, up_ptrs, down_ptrs, gate_fmt, down_fmts, gate_bias, up_bias, down_bias, act, n_experts,
             row_weights, inputs, output, k, embed_dim, inter_dim, hidden_out, hq_blocks_out);
}

TG_API void tg_moe_forward_rows(const uint8_t *const *gate_ptrs, const uint8_t *const *up_ptrs,
                                const void *const *down_ptrs, const int *down_fmts, int n_experts,
                                const float *row_weights, const float *inputs, float *output, int k, int embed_dim,
                                int inter_dim) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    moe_host(gate_ptrs, up_ptrs, down_ptrs, TG_FMT_Q4K, down_fmts, nullptr, nullptr, nullptr, TG_ACT_SILU,
             n_experts, row_weights, inputs, output, k, embed_dim, inter_dim);
}

/* tg_expert_forward_mixed down codes (csrc/libtinygiant.c:1113-1124):
 * 1 = f16, 2 = q6_K, anything else = q4_K */
static int mixed_down_fmt(int code) { return code == 1 ? TG_FMT_F16 : code == 2 ? TG_FMT_Q6K : TG_FMT_Q4K; }

TG_API void tg_expert_forward_mixed(const uint8_t *gate_q4, const uint8_t *up_q4, const void *down_data,
                                    int down_format, const float *input, float *output, float weight, int embed_dim,
                                    int inter_dim) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    const uint8_t *g1[1] = {gate_q4}, *u1[1] = {up_q4};
    const void *d1[1] = {down_data};
    int f1[1] = {mixed_down_fmt(down_format)};
    float w1[1] = {weight};
    moe_host(g1, u1, d1, TG_FMT_Q4K, f1, nullptr, nullptr, nullptr, TG_ACT_SILU, 1, w1, input, output, 1,
             embed_dim, inter_dim);
}

TG_API void tg_expert_forward(const uint8_t *q4_data, const float *input, float *output, float weight,
                              int embed_dim, int inter_dim) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    /* [gate | up | down], all Q4_K (csrc/libtinygiant.c:1040-1049) */
    const size_t gate_bytes = (size_t)inter_dim * (embed_dim / 256) * 144;
    const uint8_t *g1[1] = {q4_data}, *u1[1] = {q4_data + gate_bytes};
    const void *d1[1] = {q4_data + 2 * gate_bytes};
    int f1[1] = {TG_FMT_Q4K};
    float w1[1] = {weight};
    moe_host(g1, u1, d1, TG_FMT_Q4K, f1, nullptr, nullptr, nullptr, TG_ACT_SILU, 1, w1, input, output, 1,
             embed_dim, inter_dim);
}

TG_API void tg_expert_forward_rows(const uint8_t *gate_q4, const uint8_t *up_q4, const void *down_data,
                                   int down_format, const float *inputs, float *output, const float *weights, int k,
                                   int embed_dim, int inter_dim) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    const uint8_t *g1[1] = {gate_q4}, *u1[1] = {up_q4};
    const void *d1[1] = {down_data};
    int f1[1] = {mixed_down_fmt(down_format)};
    moe_host(g1, u1, d1, TG_FMT_Q4K, f1, nullptr, nullptr, nullptr, TG_ACT_SILU, 1, weights, inputs, output, k,
             embed_dim, inter_dim);
}

TG_API void tg_moe_forward(const uint8_t **expert_ptrs, const float *weights, int n_experts, const float *input,
                           float *output, int embed_dim, int inter_dim) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    /* csrc/libtinygiant.c:1452-1460: zero the output, then one all-Q4_K expert each */
    memset(output, 0, (size_t)embed_dim * sizeof(float));
    if (n_experts <= 0) return;
    const size_t gate_bytes = (size_t)inter_dim * (embed_dim / 256) * 144;
    std::vector<const uint8_t *> g(n_experts), u(n_experts);
    std::vector<const void *> d(n_experts);
    std::vector<int> f(n_experts, TG_FMT_Q4K);
    for (int e = 0; e < n_experts; e++) {
        g[e] = expert_ptrs[e];
        u[e] = expert_ptrs[e] + gate_bytes;
        d[e] = expert_ptrs[e] + 2 * gate_bytes;
    }
    moe_host(g.data(), u.data(), d.data(), TG_FMT_Q4K, f.data(), nullptr, nullptr, nullptr, TG_ACT_SILU,
             n_experts, weights, input, output, 1, embed_dim, inter_dim);
}

TG_API void tg_matmul(int fmt, const void *mat, const float *bias, const float *input, float *output, int nrows,
                      int ncols) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    matmul_host(fmt, mat, bias, input, output, nrows, ncols);
}

TG_API void tg_matmul_q4k(const uint8_t *q4_matrix, const float *input, float *output, int nrows, int ncols) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    matmul_host(TG_FMT_Q4K, q4_matrix, nullptr, input, output, nrows, ncols);
}

TG_API void tg_matmul_q6k(const uint8_t *q6_matrix, const float *input, float *output, int nrows, int ncols) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    matmul_host(TG_FMT_Q6K, q6_matrix, nullptr, input, output, nrows, ncols);
}

TG_API size_t tg_row_bytes(int fmt, int ncols) {
    switch (fmt) {
        case TG_FMT_Q4K: return (size_t)(ncols / 256) * 144;
        case TG_FMT_Q6K: return (size_t)(ncols / 256) * 210;
        case TG_FMT_MXFP4: return (size_t)(ncols / 32) * 17;
        case TG_FMT_Q80: return (size_t)(ncols / 32) * 34;
        default: return (size_t)ncols * 2;
    }
}

TG_API void tg_set_threads(int n) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    g_threads = n < 1 ? 1 : n;
}

TG_API int tg_get_threads(void) { return g_threads; }

/* The reference pins host pages (csrc/libtinygiant.c:1566-1571).  Here the
 * range is copied into HBM once; every later pointer inside it resolves to
 * the device copy.  Returns 0 on success, -1 if HBM is exhausted. */
TG_API int tg_mlock(const void *addr, size_t len) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    return do_register(addr, len);
}

/* ===================== tg_hip_* extensions ===================== */

TG_API const char *tg_hip_last_error(void) { return g_err; }

TG_API void tg_hip_clear_error(void) { g_err[0] = 0; }

TG_API int tg_hip_register(const void *addr, size_t len) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    return do_register(addr, len);
}

TG_API int tg_hip_unregister(const void *addr) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    auto it = g_regs.find((uintptr_t)addr);
    if (it == g_regs.end()) return -1;
    HIPCHECK(hipStreamSynchronize(g.st));
    HIPCHECK(hipFree(it->second.dev));
    g_regs.erase(it);
    g_e255_known.clear();
    return 0;
}

TG_API size_t tg_hip_registered_bytes(void) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    size_t s = 0;
    for (auto &kv : g_regs) s += kv.second.len;
    return s;
}

TG_API const void *tg_hip_device_ptr(const void *host, size_t n) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    return lookup(host, n);
}

TG_API void *tg_hip_stream(void) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    ensure_init();
    return (void *)g.st;
}

TG_API void *tg_hip_malloc(size_t n) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    ensure_init();
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, n ? n : 1);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        set_err("tg_hip_malloc(%zu): %s", n, hipGetErrorString(e));
        return nullptr;
    }
    return p;
}

TG_API void tg_hip_free(void *p) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!p) return;
    HIPCHECK(hipStreamSynchronize(g.st));
    HIPCHECK(hipFree(p));
}

TG_API void tg_hip_memcpy_h2d(void *dst, const void *src, size_t n) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    ensure_init();
    HIPCHECK(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, g.st));
    HIPCHECK(hipStreamSynchronize(g.st));
}

TG_API void tg_hip_memcpy_d2h(void *dst, const void *src, size_t n) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    ensure_init();
    HIPCHECK(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, g.st));
    HIPCHECK(hipStreamSynchronize(g.st));
}

TG_API void tg_hip_memcpy_d2d(void *dst, const void *src, size_t n, void *stream) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    ensure_init();
    HIPCHECK(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, stream ? (hipStream_t)stream : g.st));
}

TG_API void tg_hip_synchronize(void) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    ensure_init();
    HIPCHECK(hipStreamSynchronize(g.st));
    HIPCHECK(hipDeviceSynchronize());
}

/* Seeded synthetic tensor (tg_synth.h) written on the device / on the host. */
TG_API void tg_hip_synth_fill(int kind, uint64_t seed, void *dst_dev, uint64_t nbytes, void *stream) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    ensure_init();
    if (((uintptr_t)dst_dev & 7) != 0) {
        set_err("tg_hip_synth_fill: destination must be 8-byte aligned");
        return;
    }
    launch_synth_fill(kind, seed, dst_dev, nbytes, stream ? (hipStream_t)stream : g.st);
    HIPCHECK(hipGetLastError());
}

TG_API void tg_hip_synth_fill_host(int kind, uint64_t seed, void *dst, uint64_t nbytes) {
    uint8_t *p = (uint8_t *)dst;
    for (uint64_t i = 0; i < nbytes; i++) p[i] = tg_syn_byte(kind, seed, i);
}

/* q8 quantization of nrows rows of ncols floats, returned in the reference's
 * 296-byte q8_block layout (csrc/libtinygiant.c:159-164). */
TG_API void tg_hip_quantize_q8(const float *x, int ncols, int nrows, void *out_blocks) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (ncols <= 0 || ncols % 32 || nrows <= 0) {
        set_err("tg_hip_quantize_q8: ncols must be a positive multiple of 32");
        return;
    }
    ensure_init();
    Bump b;
    const size_t o_in = b.take((size_t)nrows * ncols * 4);
    const size_t o_q = b.take(q8_bytes(nrows, ncols));
    uint8_t *dev = arena(b.off);
    HIPCHECK(hipMemcpyAsync(dev + o_in, x, (size_t)nrows * ncols * 4, hipMemcpyHostToDevice, g.st));
    Q8Rows q = q8_view(dev + o_q, nrows, ncols, nullptr);
    launch_quantize((const float *)(dev + o_in), ncols, nrows, ncols, q, g.st);
    HIPCHECK(hipGetLastError());
    q8_to_blocks(q, nrows, out_blocks);
}

/* Per-sub-block integer sums of every row of a weight matrix against one
 * q8-quantized activation row, from the same decode path as the GEMV:
 * Q4_K 8 per 256-block, Q6_K 16 per 256-block, MXFP4/Q8_0 1 per 32-block. */
TG_API int tg_hip_isums(int fmt, const void *mat, int nrows, int ncols, const float *x, int32_t *out) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!fmt_ok(fmt) || fmt == TG_FMT_F16 || ncols <= 0 || ncols % 32 || nrows <= 0) {
        set_err("tg_hip_isums: bad format or shape");
        return -1;
    }
    ensure_init();
    const int nsr = (fmt == TG_FMT_Q4K) ? ncols / 256 * 8 : (fmt == TG_FMT_Q6K) ? ncols / 256 * 16 : ncols / 32;
    const size_t rb = row_bytes(fmt, ncols);
    Bump b;
    const size_t o_in = b.take((size_t)ncols * 4);
    const size_t o_q = b.take(q8_bytes(1, ncols));
    const size_t o_out = b.take((size_t)nrows * nsr * 4);
    const size_t o_m = b.take((size_t)nrows * rb);
    uint8_t *dev = arena(b.off);
    HIPCHECK(hipMemcpyAsync(dev + o_in, x, (size_t)ncols * 4, hipMemcpyHostToDevice, g.st));
    HIPCHECK(hipMemcpyAsync(dev + o_m, mat, (size_t)nrows * rb, hipMemcpyHostToDevice, g.st));
    HIPCHECK(hipMemsetAsync(dev + o_out, 0, (size_t)nrows * nsr * 4, g.st));
    Q8Rows q = q8_view(dev + o_q, 1, ncols, nullptr);
    launch_quantize((const float *)(dev + o_in), ncols, 1, ncols, q, g.st);
    launch_isums(fmt, dev + o_m, nrows, ncols, q, nsr, (int32_t *)(dev + o_out), g.st);
    HIPCHECK(hipGetLastError());
    HIPCHECK(hipMemcpyAsync(out, dev + o_out, (size_t)nrows * nsr * 4, hipMemcpyDeviceToHost, g.st));
    HIPCHECK(hipStreamSynchronize(g.st));
    return nsr;
}

/* ---- device-resident MoE plans (pointers already in HBM) ---- */

struct tg_hip_moe_plan {
    HostPlan h;
    Layout L;
    uint8_t *dev;
    MoeArgs a;
};

TG_API tg_hip_moe_plan *tg_hip_moe_plan_create(const void *const *gate_dev, const void *const *up_dev,
                                               const void *const *down_dev, int gate_fmt, const int *down_fmts,
                                               const float *const *gate_bias_dev, const float *const *up_bias_dev,
                                               const float *const *down_bias_dev, int act, int n_experts,
                                               const float *row_weights, int k, int embed_dim, int inter_dim) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!validate_moe(gate_fmt, down_fmts, n_experts, k, embed_dim, inter_dim, act)) return nullptr;
    if (n_experts == 0 || k == 0) {
        set_err("tg_hip_moe_plan_create: empty plan");
        return nullptr;
    }
    ensure_init();
    tg_hip_moe_plan *p = new tg_hip_moe_plan();
    HostPlan &h = p->h;
    h.n = n_experts;
    h.k = k;
    h.D = embed_dim;
    h.I = inter_dim;
    h.act = act;
    h.gate_fmt = gate_fmt;
    h.down_fmt.assign(down_fmts, down_fmts + n_experts);
    build_pairs(h, row_weights);
    h.has_gb = gate_bias_dev != nullptr;
    h.has_ub = up_bias_dev != nullptr;
    h.has_db = down_bias_dev != nullptr;
    if (h.has_gb != h.has_ub) {
        set_err("moe plan: gate and up biases must both be given or both be NULL");
        return nullptr;
    }
    for (int e = 0; e < n_experts; e++) {
        h.gate.push_back((uint64_t)(uintptr_t)gate_dev[e]);
        h.up.push_back((uint64_t)(uintptr_t)up_dev[e]);
        h.down.push_back((uint64_t)(uintptr_t)down_dev[e]);
        h.gbias.push_back(h.has_gb ? (uint64_t)(uintptr_t)gate_bias_dev[e] : 0);
        h.ubias.push_back(h.has_ub ? (uint64_t)(uintptr_t)up_bias_dev[e] : 0);
        h.dbias.push_back(h.has_db ? (uint64_t)(uintptr_t)down_bias_dev[e] : 0);
    }
    p->L = plan_layout(h);
    HIPCHECK(hipMalloc(&p->dev, p->L.total));
    std::vector<uint8_t> img(p->L.tables_len);
    p->a = plan_args(h, p->L, p->dev, img.data());
    /* the caller's device matrices, scanned once (the MFMA threshold may
     * change after the plan is made) */
    const auto mats = mx_matrices(h);
    p->a.mx_e255 = mx_any_e255(mats, std::vector<char>(mats.size(), 0)) ? 1 : 0;
    HIPCHECK(hipMemcpy(p->dev + p->L.tables, img.data(), img.size(), hipMemcpyHostToDevice));
    HIPCHECK(hipMemset(p->dev + p->L.ctr, 0, (size_t)moe_ctr_words(h.D) * 4));
    return p;
}

/* Queues the layer on `stream` (null = the library stream): quantize inputs,
 * gate/up + act, quantize hidden, down, combine into `output` (accumulated).
 * Launches only kernels, so it can be captured into a HIP graph. */
TG_API void tg_hip_moe_plan_run(tg_hip_moe_plan *p, const float *inputs_dev, float *output_dev, void *stream) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!p) return;
    if (p->h.P == 0) return;
    MoeArgs a = p->a;
    a.xin = inputs_dev;
    a.xq.f = inputs_dev;
    a.out = output_dev;
    launch_moe(a, p->h.fmts_present.data(), (int)p->h.fmts_present.size(), stream ? (hipStream_t)stream : g.st);
    HIPCHECK(hipGetLastError());
}

TG_API int tg_hip_moe_plan_pairs(const tg_hip_moe_plan *p) { return p ? p->h.P : 0; }

TG_API void tg_hip_moe_plan_destroy(tg_hip_moe_plan *p) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!p) return;
    HIPCHECK(hipStreamSynchronize(g.st));
    HIPCHECK(hipFree(p->dev));
    delete p;
}

/* y[j][r] = dot(W[r], x_j) + bias[r] for k rows of device-resident input. */
TG_API void tg_hip_matmul_dev(int fmt, const void *mat_dev, const float *bias_dev, const float *inputs_dev,
                              float *outputs_dev, int nrows, int ncols, int k, void *scratch_dev, void *stream) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!fmt_ok(fmt) || ncols <= 0 || ncols % 32 || nrows <= 0 || k <= 0) {
        set_err("tg_hip_matmul_dev: bad format or shape");
        return;
    }
    ensure_init();
    hipStream_t st = stream ? (hipStream_t)stream : g.st;
    Q8Rows q = q8_view((uint8_t *)scratch_dev, k, ncols, inputs_dev);
    if (fmt != TG_FMT_F16) launch_quantize(inputs_dev, ncols, k, ncols, q, st);
    launch_gemv(fmt, (const uint8_t *)mat_dev, nrows, ncols, bias_dev, q, k, outputs_dev, nrows, st);
    HIPCHECK(hipGetLastError());
}

TG_API size_t tg_hip_matmul_scratch_bytes(int k, int ncols) { return q8_bytes(k, ncols); }

/* Sets up the library on the current device (its stream and the device
 * address of the fixed scratch); every other entry point does it on first
 * use, tg_hip_matmul_dev_noalloc requires it. */
TG_API void tg_hip_init(void) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    ensure_init();
}

static void release_upload_buffers();
static void release_marks();

/* Waits for the device and releases everything the library holds: its
 * stream, the device arena, the pinned and coherent host rows, the ticket
 * words, the file-upload buffers and the timing marks.  Objects the caller
 * created (plans, decode steps, device arrays) stay theirs to destroy first.
 * A later call re-initialises the library. */
TG_API void tg_hip_shutdown(void) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!g.ready) return;
    HIPCHECK(hipStreamSynchronize(g.st));
    HIPCHECK(hipDeviceSynchronize());
    release_upload_buffers();
    release_marks();
    if (g.arena) HIPCHECK(hipFree(g.arena));
    if (g.tickets) HIPCHECK(hipFree(g.tickets));
    if (g.pin) HIPCHECK(hipHostFree(g.pin));
    if (g.io) HIPCHECK(hipHostFree(g.io));
    HIPCHECK(hipStreamDestroy(g.st));
    g = Ctx();
}

/* tg_hip_matmul_dev without a workspace and without any allocation: the q8
 * rows of the inputs go to the library's fixed device scratch, which holds
 * tg_hip_matmul_noalloc_max_bytes() bytes (k * ceil(ncols/256) * 360 bytes
 * are needed).  For callers that cannot allocate (HIP graph capture, serving
 * loops).  Needs tg_hip_init() first.  Calls on one GPU share the scratch:
 * calls that overlap in time on one GPU (other streams, other threads'
 * queued work) race. */
TG_API void tg_hip_matmul_dev_noalloc(int fmt, const void *mat_dev, const float *bias_dev, const float *inputs_dev,
                                      float *outputs_dev, int nrows, int ncols, int k, void *stream) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!fmt_ok(fmt) || ncols <= 0 || ncols % 32 || nrows <= 0 || k <= 0) {
        set_err("tg_hip_matmul_dev_noalloc: bad format or shape");
        return;
    }
    if (!g.ready) {
        set_err("tg_hip_matmul_dev_noalloc: call tg_hip_init() first");
        return;
    }
    if (q8_bytes(k, ncols) > NOALLOC_SCRATCH_BYTES) {
        set_err("tg_hip_matmul_dev_noalloc: %d rows of %d columns need %zu scratch bytes, the fixed scratch holds %zu",
                k, ncols, q8_bytes(k, ncols), NOALLOC_SCRATCH_BYTES);
        return;
    }
    hipStream_t st = stream ? (hipStream_t)stream : g.st;
    Q8Rows q = q8_view(g.scratch, k, ncols, inputs_dev);
    if (fmt != TG_FMT_F16) launch_quantize(inputs_dev, ncols, k, ncols, q, st);
    launch_gemv(fmt, (const uint8_t *)mat_dev, nrows, ncols, bias_dev, q, k, outputs_dev, nrows, st);
    HIPCHECK(hipGetLastError());
}

TG_API size_t tg_hip_matmul_noalloc_max_bytes(void) { return NOALLOC_SCRATCH_BYTES; }

/* ---- decode attention (tg_attention_v2, csrc/libtinygiant.c:939-983) ----
 * Scratch: q8 of the input | Q, K, V projections | chunk partials |
 * attention output | its q8 | one ticket counter per KV head. */
struct AttnLayout {
    size_t xq, qkv, part, att, aq, ctr, total;
};

static AttnLayout attn_layout(int embed_dim, int n_heads, int n_kv, int head_dim, int kv_max) {
    AttnLayout L;
    Bump b;
    const size_t q_dim = (size_t)n_heads * head_dim, kv_dim = (size_t)n_kv * head_dim;
    const size_t nch = ((size_t)kv_max + ATTN_CHUNK - 1) / ATTN_CHUNK;
    L.xq = b.take(q8_bytes(1, embed_dim));
    L.qkv = b.take((q_dim + 2 * kv_dim) * 4);
    L.part = b.take((size_t)n_heads * nch * (head_dim + 2) * 4);
    L.att = b.take(q_dim * 4);
    L.aq = b.take(q8_bytes(1, (int)q_dim));
    L.ctr = b.take((size_t)n_kv * 4);
    L.total = b.off;
    return L;
}

static bool attn_validate(const char *who, int fmt_q, int fmt_k, int fmt_v, int fmt_o, const float *q_norm_w,
                          const float *k_norm_w, int kv_len, int kv_max, int window, int embed_dim, int n_heads,
                          int n_kv, int head_dim, int pos) {
    if (!fmt_ok(fmt_q) || !fmt_ok(fmt_k) || !fmt_ok(fmt_v) || !fmt_ok(fmt_o)) {
        set_err("%s: unsupported weight format", who);
        return false;
    }
    if (embed_dim <= 0 || embed_dim % 32 || n_heads <= 0 || n_kv <= 0 || n_heads % n_kv ||
        n_heads / n_kv > ATTN_MAX_GQA || head_dim <= 0 || head_dim % 4 || head_dim > ATTN_MAX_HEAD_DIM ||
        (n_heads * head_dim) % 32) {
        set_err("%s: unsupported shape (embed_dim %% 32 == 0, head_dim %% 4 == 0 and <= %d, n_heads / n_kv_heads "
                "integral and <= %d)", who, ATTN_MAX_HEAD_DIM, ATTN_MAX_GQA);
        return false;
    }
    if (kv_len < 0 || kv_len >= kv_max || kv_max > ATTN_CHUNK * ATTN_MAX_CHUNKS || window < 0 || pos < 0) {
        set_err("%s: need 0 <= kv_len < kv_max <= %d, window >= 0, pos >= 0", who, ATTN_CHUNK * ATTN_MAX_CHUNKS);
        return false;
    }
    if (q_norm_w && !k_norm_w) {
        set_err("%s: q_norm_w without k_norm_w (the reference dereferences it)", who);
        return false;
    }
    return true;
}

/* every pointer on the device; rope rows are the tables at pos */
static void attn_run(int fmt_q, int fmt_k, int fmt_v, int fmt_o, const void *wq, const void *wk, const void *wv,
                     const void *wo, const float *bq, const float *bk, const float *bv, const float *bo,
                     const float *q_norm_w, const float *k_norm_w, const float *sinks, float *kv_k, float *kv_v,
                     int kv_len, int kv_max, int window, const float *rope_cos_row, const float *rope_sin_row,
                     const float *input, float *output, int embed_dim, int n_heads, int n_kv, int head_dim, float eps,
                     float *att_out, uint8_t *scratch, hipStream_t st) {
    const AttnLayout L = attn_layout(embed_dim, n_heads, n_kv, head_dim, kv_max);
    const int q_dim = n_heads * head_dim, kv_dim = n_kv * head_dim;
    float *qkv = (float *)(scratch + L.qkv);
    unsigned *ctr = (unsigned *)(scratch + L.ctr);
    /* Q, K and V projections */
    const int fmts[3] = {fmt_q, fmt_k, fmt_v};
    const GemvJob all[3] = {{(const uint8_t *)wq, bq, qkv, q_dim, q_dim},
                            {(const uint8_t *)wk, bk, qkv + q_dim, kv_dim, kv_dim},
                            {(const uint8_t *)wv, bv, qkv + q_dim + kv_dim, kv_dim, kv_dim}};
    const bool fused_x = gemv_q8x_ok(fmts, 3, embed_dim);
    if (fused_x) {
        /* Q4_K / Q6_K: q8 of the input inside the one projection launch,
         * which also clears the ticket counters of the partial kernel */
        const GemvJobs jobs = {{all[0], all[1], all[2]}};
        launch_gemv_q8x(fmts, jobs, 3, embed_dim, input, ctr, n_kv, st);
    } else {
        /* q8 once, then one launch per distinct format */
        Q8Rows xq = q8_view(scratch + L.xq, 1, embed_dim, input);
        if (fmt_q != TG_FMT_F16 || fmt_k != TG_FMT_F16 || fmt_v != TG_FMT_F16)
            launch_quantize(input, embed_dim, 1, embed_dim, xq, st);
        for (int i = 0; i < 3; i++) {
            bool first = true;
            for (int j = 0; j < i; j++) first &= fmts[j] != fmts[i];
            if (!first) continue;
            GemvJobs jobs;
            int nj = 0;
            for (int j = i; j < 3; j++)
                if (fmts[j] == fmts[i]) jobs.j[nj++] = all[j];
            launch_gemv_multi(fmts[i], jobs, nj, embed_dim, xq, 1, st);
        }
    }
    float *att = (float *)(scratch + L.att);
    Q8Rows aq = q8_view(scratch + L.aq, 1, q_dim, att);
    /* attention; q8 of its output fused into the combine where the block
     * layout allows, and the combine into the partial kernel for short spans
     * (its counters are cleared by the fused projection launch) */
    const bool fuse_q8 = fmt_o != TG_FMT_F16 && attention_combine_q8_ok(n_heads, head_dim);
    launch_attention_core(qkv, q_norm_w, k_norm_w, sinks, kv_k, kv_v, kv_len, kv_max, window, rope_cos_row,
                          rope_sin_row, n_heads, n_kv, head_dim, eps, (float *)(scratch + L.part), att,
                          fuse_q8 ? &aq : nullptr, st, fused_x ? ctr : nullptr);
    if (fmt_o != TG_FMT_F16 && !fuse_q8) launch_quantize(att, q_dim, 1, q_dim, aq, st);
    launch_gemv(fmt_o, (const uint8_t *)wo, embed_dim, q_dim, bo, aq, 1, output, embed_dim, st);
    if (att_out) HIPCHECK(hipMemcpyAsync(att_out, att, (size_t)q_dim * 4, hipMemcpyDeviceToDevice, st));
}

TG_API size_t tg_hip_attention_scratch_bytes(int embed_dim, int n_heads, int n_kv_heads, int head_dim, int kv_max) {
    if (embed_dim <= 0 || n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 || kv_max <= 0) return 0;
    return attn_layout(embed_dim, n_heads, n_kv_heads, head_dim, kv_max).total;
}

TG_API void tg_hip_attention_dev(int fmt_q, int fmt_k, int fmt_v, int fmt_o, const void *wq, const void *wk,
                                 const void *wv, const void *wo, const float *bq, const float *bk, const float *bv,
                                 const float *bo, const float *q_norm_w, const float *k_norm_w, const float *sinks,
                                 float *kv_k, float *kv_v, int kv_len, int kv_max, int window, const float *rope_cos,
                                 const float *rope_sin, const float *input, float *output, int embed_dim, int n_heads,
                                 int n_kv_heads, int head_dim, int pos, float eps, float *att_out, void *scratch,
                                 void *stream) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!attn_validate("tg_hip_attention_dev", fmt_q, fmt_k, fmt_v, fmt_o, q_norm_w, k_norm_w, kv_len, kv_max, window,
                       embed_dim, n_heads, n_kv_heads, head_dim, pos))
        return;
    if (!wq || !wk || !wv || !wo || !kv_k || !kv_v || !rope_cos || !rope_sin || !input || !output || !scratch) {
        set_err("tg_hip_attention_dev: null weight, cache, table, input, output or scratch pointer");
        return;
    }
    if (((uintptr_t)kv_k | (uintptr_t)kv_v) & 15) {
        set_err("tg_hip_attention_dev: kv_k and kv_v must be 16-byte aligned");
        return;
    }
    ensure_init();
    const size_t half = (size_t)head_dim / 2;
    attn_run(fmt_q, fmt_k, fmt_v, fmt_o, wq, wk, wv, wo, bq, bk, bv, bo, q_norm_w, k_norm_w, sinks, kv_k, kv_v, kv_len,
             kv_max, window, rope_cos + (size_t)pos * half, rope_sin + (size_t)pos * half, input, output, embed_dim,
             n_heads, n_kv_heads, head_dim, eps, att_out, (uint8_t *)scratch, stream ? (hipStream_t)stream : g.st);
    HIPCHECK(hipGetLastError());
}

/* tg_attention_v2 with the reference's host pointers (csrc/libtinygiant.c:939-983).
 * Registered ranges (tg_mlock) are used in place: weights, and the KV arrays,
 * whose device copy the kernels update; everything else is staged for the
 * call.  The new K and V rows are also written into the host arrays at kv_len
 * and output is overwritten, as the reference does. */
TG_API void tg_attention_v2(int fmt_q, int fmt_k, int fmt_v, int fmt_o, const void *wq, const void *wk,
                            const void *wv, const void *wo, const float *bq, const float *bk, const float *bv,
                            const float *bo, const float *q_norm_w, const float *k_norm_w, const float *sinks,
                            float *kv_k, float *kv_v, int kv_len, int kv_max, int window, const float *rope_cos,
                            const float *rope_sin, const float *input, float *output, int embed_dim, int n_heads,
                            int n_kv_heads, int head_dim, int pos, float eps) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!attn_validate("tg_attention_v2", fmt_q, fmt_k, fmt_v, fmt_o, q_norm_w, k_norm_w, kv_len, kv_max, window,
                       embed_dim, n_heads, n_kv_heads, head_dim, pos))
        return;
    ensure_init();
    const int q_dim = n_heads * head_dim, kv_dim = n_kv_heads * head_dim;
    const size_t half = (size_t)head_dim / 2;
    const AttnLayout AL = attn_layout(embed_dim, n_heads, n_kv_heads, head_dim, kv_max);
    Bump bump;
    bump.off = AL.total;
    const size_t io_in = bump.take((size_t)embed_dim * 4), io_out = bump.take((size_t)embed_dim * 4);
    Stager sg;
    sg.bump = &bump;
    struct Ptr {
        uintptr_t v;
        bool staged;
    };
    auto res = [&](const void *p, size_t n) -> Ptr {
        Ptr r{0, false};
        if (p) r.v = sg.resolve(p, n, &r.staged);
        return r;
    };
    const size_t cache_bytes = (size_t)n_kv_heads * kv_max * head_dim * 4;
    Ptr pq = res(wq, (size_t)q_dim * row_bytes(fmt_q, embed_dim)), pk = res(wk, (size_t)kv_dim * row_bytes(fmt_k, embed_dim));
    Ptr pv = res(wv, (size_t)kv_dim * row_bytes(fmt_v, embed_dim)), po = res(wo, (size_t)embed_dim * row_bytes(fmt_o, q_dim));
    Ptr pbq = res(bq, (size_t)q_dim * 4), pbk = res(bk, (size_t)kv_dim * 4), pbv = res(bv, (size_t)kv_dim * 4);
    Ptr pbo = res(bo, (size_t)embed_dim * 4);
    Ptr pqn = res(q_norm_w, (size_t)head_dim * 4), pkn = res(k_norm_w, (size_t)head_dim * 4);
    Ptr psk = res(sinks, (size_t)n_heads * 4);
    Ptr pkk = res(kv_k, cache_bytes), pkv = res(kv_v, cache_bytes);
    Ptr prc = res(rope_cos + (size_t)pos * half, half * 4), prs = res(rope_sin + (size_t)pos * half, half * 4);
    uint8_t *dev = arena(bump.off);
    auto dp = [&](const Ptr &p) -> void * {
        if (!p.v && !p.staged) return nullptr;
        return p.staged ? (void *)(dev + p.v) : (void *)p.v;
    };
    for (auto &it : sg.items) HIPCHECK(hipMemcpyAsync(dev + it.off, it.host, it.n, hipMemcpyHostToDevice, g.st));
    HIPCHECK(hipMemcpyAsync(dev + io_in, input, (size_t)embed_dim * 4, hipMemcpyHostToDevice, g.st));
    float *dkk = (float *)dp(pkk), *dkv = (float *)dp(pkv);
    attn_run(fmt_q, fmt_k, fmt_v, fmt_o, dp(pq), dp(pk), dp(pv), dp(po), (const float *)dp(pbq), (const float *)dp(pbk),
             (const float *)dp(pbv), (const float *)dp(pbo), (const float *)dp(pqn), (const float *)dp(pkn),
             (const float *)dp(psk), dkk, dkv, kv_len, kv_max, window, (const float *)dp(prc), (const float *)dp(prs),
             (const float *)(dev + io_in), (float *)(dev + io_out), embed_dim, n_heads, n_kv_heads, head_dim, eps,
             nullptr, dev, g.st);
    HIPCHECK(hipGetLastError());
    /* the new rows back into the host arrays, the output */
    for (int h = 0; h < n_kv_heads; h++) {
        const size_t off = ((size_t)h * kv_max + kv_len) * head_dim;
        HIPCHECK(hipMemcpyAsync(kv_k + off, dkk + off, (size_t)head_dim * 4, hipMemcpyDeviceToHost, g.st));
        HIPCHECK(hipMemcpyAsync(kv_v + off, dkv + off, (size_t)head_dim * 4, hipMemcpyDeviceToHost, g.st));
    }
    HIPCHECK(hipMemcpyAsync(output, dev + io_out, (size_t)embed_dim * 4, hipMemcpyDeviceToHost, g.st));
    HIPCHECK(hipStreamSynchronize(g.st));
}

/* ---- file -> HBM upload (the expert-cache loader's native part) ----
 * Two pinned staging buffers: while one is being copied to the device, the
 * next chunk of the file is read into the other, by UP_THREADS threads each
 * reading a contiguous share (one thread copying out of the page cache runs
 * at about 9 GB/s, well under the host-to-device link). */
static uint8_t *g_up_buf[2] = {nullptr, nullptr};
static size_t g_up_cap = 0;
static hipEvent_t g_up_ev[2];
static const int UP_THREADS = 8;

static void release_upload_buffers() {
    for (int i = 0; i < 2; i++) {
        if (!g_up_buf[i]) continue;
        HIPCHECK(hipEventSynchronize(g_up_ev[i]));
        HIPCHECK(hipEventDestroy(g_up_ev[i]));
        HIPCHECK(hipHostFree(g_up_buf[i]));
        g_up_buf[i] = nullptr;
    }
    g_up_cap = 0;
}

/* Reads n bytes at file offset off into dst; returns how many bytes were read
 * before the first share that ended early (n when none did). */
static uint64_t read_span(int fd, uint8_t *dst, uint64_t n, uint64_t off) {
    const uint64_t min_share = 1u << 20;
    int t = (int)std::min<uint64_t>(UP_THREADS, std::max<uint64_t>(1, n / min_share));
    const uint64_t share = (n + t - 1) / t;
    std::vector<uint64_t> got(t, 0);
    auto work = [&](int i) {
        const uint64_t b = (uint64_t)i * share, e = std::min(n, b + share);
        uint64_t p = b;
        while (p < e) {
            const ssize_t r = pread(fd, dst + p, e - p, (off_t)(off + p));
            if (r <= 0) break;
            p += (uint64_t)r;
        }
        got[i] = p - b;
    };
    std::vector<std::thread> th;
    for (int i = 1; i < t; i++) th.emplace_back(work, i);
    work(0);
    for (auto &x : th) x.join();
    uint64_t done = 0;
    for (int i = 0; i < t; i++) {
        done += got[i];
        if (got[i] < std::min(n, (uint64_t)(i + 1) * share) - (uint64_t)i * share) break;
    }
    return done;
}

TG_API int64_t tg_hip_upload_file(const char *path, uint64_t file_offset, uint64_t nbytes, void *dev_dst,
                                  uint64_t chunk_bytes) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!path || !dev_dst) {
        set_err("tg_hip_upload_file: null path or destination");
        return -1;
    }
    ensure_init();
    if (chunk_bytes < (1u << 20)) chunk_bytes = 1u << 20;
    if (chunk_bytes > g_up_cap) {
        for (int i = 0; i < 2; i++) {
            if (g_up_buf[i]) {
                HIPCHECK(hipEventSynchronize(g_up_ev[i]));
                HIPCHECK(hipHostFree(g_up_buf[i]));
            } else {
                HIPCHECK(hipEventCreateWithFlags(&g_up_ev[i], hipEventDisableTiming));
                HIPCHECK(hipEventRecord(g_up_ev[i], g.st));
            }
            if (hipHostMalloc((void **)&g_up_buf[i], chunk_bytes, hipHostMallocDefault) != hipSuccess) {
                (void)hipGetLastError();
                g_up_buf[i] = nullptr;
                g_up_cap = 0;
                set_err("tg_hip_upload_file: cannot allocate %llu bytes of pinned memory",
                        (unsigned long long)chunk_bytes);
                return -1;
            }
        }
        g_up_cap = chunk_bytes;
    }
    const int fd = open(path, O_RDONLY);
    if (fd < 0) {
        set_err("tg_hip_upload_file: cannot open %s", path);
        return -1;
    }
    uint64_t done = 0;
    int slot = 0;
    while (done < nbytes) {
        const uint64_t n = std::min<uint64_t>(g_up_cap, nbytes - done);
        HIPCHECK(hipEventSynchronize(g_up_ev[slot]));   /* the copy that last used this buffer */
        const uint64_t got = read_span(fd, g_up_buf[slot], n, file_offset + done);
        if (got < n) {
            close(fd);
            HIPCHECK(hipStreamSynchronize(g.st));
            set_err("tg_hip_upload_file: %s ends at %llu, %llu bytes short", path,
                    (unsigned long long)(file_offset + done + got), (unsigned long long)(nbytes - done - got));
            return -1;
        }
        HIPCHECK(hipMemcpyAsync((uint8_t *)dev_dst + done, g_up_buf[slot], n, hipMemcpyHostToDevice, g.st));
        HIPCHECK(hipEventRecord(g_up_ev[slot], g.st));
        done += n;
        slot ^= 1;
    }
    close(fd);
    HIPCHECK(hipStreamSynchronize(g.st));
    return (int64_t)done;
}

/* ---- router ---- */
TG_API size_t tg_hip_route_scratch_bytes(int k, int n_experts) { return (size_t)k * n_experts * 4; }

static void route_dev(const char *name, const float *router_dev, const float *bias_dev, const float *x_dev, int k,
                      int n_experts, int dim, int top_k, const uint8_t *resident_dev, int32_t *idx_dev, float *w_dev,
                      void *scratch_dev, void *stream) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!router_dev || !x_dev || !idx_dev || !w_dev || !scratch_dev || k <= 0 || dim <= 0 || n_experts <= 0 ||
        n_experts > 256 || top_k <= 0 || top_k > 64 || top_k > n_experts) {
        set_err("%s: bad arguments (n_experts <= 256, 1 <= top_k <= 64)", name);
        return;
    }
    ensure_init();
    launch_route(router_dev, bias_dev, x_dev, k, n_experts, dim, top_k, resident_dev, (float *)scratch_dev, idx_dev,
                 w_dev, stream ? (hipStream_t)stream : g.st);
    HIPCHECK(hipGetLastError());
}

TG_API void tg_hip_route_dev(const float *router_dev, const float *bias_dev, const float *x_dev, int k, int n_experts,
                             int dim, int top_k, int32_t *idx_dev, float *w_dev, void *scratch_dev, void *stream) {
    route_dev("tg_hip_route_dev", router_dev, bias_dev, x_dev, k, n_experts, dim, top_k, nullptr, idx_dev, w_dev,
              scratch_dev, stream);
}

TG_API void tg_hip_route_restricted_dev(const float *router_dev, const float *bias_dev, const float *x_dev, int k,
                                        int n_experts, int dim, int top_k, const uint8_t *resident_dev,
                                        int32_t *idx_dev, float *w_dev, void *scratch_dev, void *stream) {
    if (!resident_dev) {
        set_err("tg_hip_route_restricted_dev: no resident mask");
        return;
    }
    route_dev("tg_hip_route_restricted_dev", router_dev, bias_dev, x_dev, k, n_experts, dim, top_k, resident_dev,
              idx_dev, w_dev, scratch_dev, stream);
}

/* ---- output head with fused argmax ----
 * Scratch: q8 rows | 16 argmax keys | RMSNorm'd rows | logits (only when the
 * format has no fused kernel and the caller passes no logits buffer). */
static size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

TG_API size_t tg_hip_head_scratch_bytes(int k, int nrows, int ncols) {
    if (k <= 0 || nrows <= 0 || ncols <= 0) return 0;
    return align256(q8_bytes(k, ncols)) + align256(HEAD_KEY_WORDS * 8) + align256((size_t)k * ncols * 4) +
           align256((size_t)k * nrows * 4);
}

TG_API void tg_hip_head_argmax_dev(int fmt, const void *mat_dev, const float *inputs_dev, const float *norm_w_dev,
                                   float eps, int k, int nrows, int ncols, float *logits_dev, int32_t *argmax_dev,
                                   float *maxval_dev, void *scratch_dev, void *stream) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!fmt_ok(fmt) || ncols <= 0 || ncols % 32 || nrows <= 0 || k <= 0 || k > 16 || !argmax_dev || !scratch_dev ||
        (norm_w_dev && !rms_norm_fits(ncols))) {
        set_err("tg_hip_head_argmax_dev: bad format, shape or arguments (1 <= k <= 16, ncols <= 16384 with a norm)");
        return;
    }
    ensure_init();
    hipStream_t st = stream ? (hipStream_t)stream : g.st;
    uint8_t *sp = (uint8_t *)scratch_dev;
    uint8_t *q8p = sp;
    unsigned long long *keys = (unsigned long long *)(sp + align256(q8_bytes(k, ncols)));
    float *normed = (float *)((uint8_t *)keys + align256(HEAD_KEY_WORDS * 8));
    float *lg_scratch = (float *)((uint8_t *)normed + align256((size_t)k * ncols * 4));
    const float *xin = norm_w_dev ? normed : inputs_dev;
    Q8Rows q = q8_view(q8p, k, ncols, xin);
    /* the fused kernel's keys and finish counter start at zero: the q8
     * kernel before it clears them */
    const bool fast = head_fast_ok(fmt, ncols, nrows, k);
    unsigned long long *clr = fast ? keys : nullptr;
    if (norm_w_dev) {
        /* RMSNorm fused with q8 of the normed rows */
        if (fmt != TG_FMT_F16) {
            launch_rms_norm_q8(inputs_dev, norm_w_dev, normed, k, ncols, eps, q, st, clr, HEAD_KEY_WORDS);
        } else {
            launch_rms_norm(inputs_dev, norm_w_dev, normed, k, ncols, eps, st);
        }
    } else if (fmt != TG_FMT_F16) {
        launch_quantize(xin, ncols, k, ncols, q, st, clr, HEAD_KEY_WORDS);
    }
    if (fast) {
        launch_head_q6k((const uint8_t *)mat_dev, nrows, q, k, logits_dev, keys, argmax_dev, maxval_dev, st);
    } else {
        float *lg = logits_dev ? logits_dev : lg_scratch;
        launch_gemv(fmt, (const uint8_t *)mat_dev, nrows, ncols, nullptr, q, k, lg, nrows, st);
        launch_argmax_rows(lg, nrows, k, keys, st);
        launch_argmax_finish(keys, k, argmax_dev, maxval_dev, st);
    }
    HIPCHECK(hipGetLastError());
}

TG_API void tg_hip_rms_norm_dev(const float *x_dev, const float *w_dev, float *out_dev, int nrows, int n, float eps,
                                void *stream) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!x_dev || !out_dev || nrows <= 0 || !rms_norm_fits(n)) {
        set_err("tg_hip_rms_norm_dev: bad arguments (1 <= n <= 16384)");
        return;
    }
    ensure_init();
    launch_rms_norm(x_dev, w_dev, out_dev, nrows, n, eps, stream ? (hipStream_t)stream : g.st);
    HIPCHECK(hipGetLastError());
}

/* ---- device-resident multi-layer decode step ----
 * h <- h + MoE_l(RMSNorm(h)) for l = 0..L-1 on k rows of width D, the chain
 * tinygiant/engine.py:281-282,335-341 runs per layer (RMSNorm weight 1 when
 * norm_w is NULL).  The launch sequence is captured once into a HIP graph
 * and replayed by tg_hip_decode_run. */

struct tg_hip_decode {
    std::vector<tg_hip_moe_plan *> plans;
    std::vector<const float *> norm_w;
    int L = 0, D = 0, k = 0, mode = 0;
    float eps = 1e-6f;
    float *h = nullptr;
    float *x = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    /* persistent mode: kind 0 the Qwen3 kernel (layers), 1 the gpt-oss
     * kernel (layers_mx) */
    int kind = 0;
    DecodeLayer *layers = nullptr;
    DecodeLayerMx *layers_mx = nullptr;
    float *hidden = nullptr;
    unsigned *sync = nullptr;    /* word 0: abort flag; word 1: the kernels' launch epoch */
    int grid = 0;
    /* mode 2: the persistent kernel as one cooperative graph node (a graph
     * launch costs ~6 us against ~19 us for a cooperative launch); its
     * arguments are fixed, and a setter that changes one marks it stale */
    hipGraph_t cgraph = nullptr;
    hipGraphExec_t cexec = nullptr;
    bool cstale = false;
    uint8_t *debug = nullptr;
    uint64_t *times = nullptr;
    uint8_t *qdown = nullptr;    /* Qwen3 kernel: the layers' down matrices in the row-group layout */
    uint8_t *mxgu = nullptr;     /* gpt-oss kernel: the layers' gate and up matrices in the wave-segment layout */
    unsigned *place = nullptr;   /* Qwen3 kernel: HW_REG_XCC_ID of each workgroup, last launch */
    int pol = 0;                 /* persistent kernels: 1 = every exchange slot stored device-coherently */
    int placement_bad = 0;       /* a launch ran with workgroup g off XCD g % 8 */
    RowsLayer *layers_rows = nullptr;   /* kind 2, the multi-row kernel: its layers */
    size_t rows_rec = 0;                /* ... and the bytes of its per-layer debug record */
};

/* the gpt-oss kernel covers k = 1 steps of 4 MXFP4 experts of 2880 x 2880
 * with the clamped SwiGLU (biases optional) */
static bool persistent_mx_ok(tg_hip_decode *d, std::vector<DecodeLayerMx> &out) {
    for (int l = 0; l < d->L; l++) {
        const HostPlan &h = d->plans[l]->h;
        if (d->plans[l]->a.mx_e255) {
            set_err("persistent decode: layer %d has an MXFP4 scale byte of 255, which the step's block-scaled MFMA "
                    "cannot apply as 2^127; use mode 0 or 1 (per-layer kernels)", l);
            return false;
        }
        if (h.k != 1 || h.D != DECODE_MX_D || h.I != DECODE_MX_D || h.gate_fmt != TG_FMT_MXFP4 ||
            h.act != TG_ACT_GPTOSS) {
            set_err("persistent decode: layer %d is not a 1-row gpt-oss MXFP4 step of %dx%d", l, DECODE_MX_D,
                    DECODE_MX_D);
            return false;
        }
        DecodeLayerMx ly;
        memset(&ly, 0, sizeof ly);
        for (int e = 0; e < h.n; e++) {
            if (h.p_off[e + 1] == h.p_off[e]) continue;
            if (ly.n >= DECODE_MX_E || h.down_fmt[e] != TG_FMT_MXFP4) {
                set_err("persistent decode: layer %d needs %d active experts with MXFP4 down", l, DECODE_MX_E);
                return false;
            }
            ly.gate[ly.n] = (const uint8_t *)(uintptr_t)h.gate[e];
            ly.up[ly.n] = (const uint8_t *)(uintptr_t)h.up[e];
            ly.down[ly.n] = (const uint8_t *)(uintptr_t)h.down[e];
            ly.gb[ly.n] = h.has_gb ? (const float *)(uintptr_t)h.gbias[e] : nullptr;
            ly.ub[ly.n] = h.has_ub ? (const float *)(uintptr_t)h.ubias[e] : nullptr;
            ly.db[ly.n] = h.has_db ? (const float *)(uintptr_t)h.dbias[e] : nullptr;
            ly.w[ly.n] = h.p_w[h.p_off[e]];
            ly.n++;
        }
        if (ly.n != DECODE_MX_E) {
            set_err("persistent decode: layer %d has %d active experts, the kernel runs exactly %d", l, ly.n,
                    DECODE_MX_E);
            return false;
        }
        ly.norm_w = d->norm_w.empty() ? nullptr : d->norm_w[l];
        out.push_back(ly);
    }
    return true;
}

/* the Qwen3 kernel covers k = 1 steps of the Qwen expert shape */
static bool persistent_ok(tg_hip_decode *d, std::vector<DecodeLayer> &out) {
    const DecodeShape sh = decode_qwen_shape();
    for (int l = 0; l < d->L; l++) {
        const HostPlan &h = d->plans[l]->h;
        if (h.k != 1 || h.D != sh.D || h.I != sh.I || h.gate_fmt != sh.gate_fmt || h.act != TG_ACT_SILU ||
            h.has_gb || h.has_ub || h.has_db) {
            set_err("persistent decode: layer %d is not a 1-row SiLU Q4_K gate/up step of %dx%d without biases", l,
                    sh.D, sh.I);
            return false;
        }
        DecodeLayer ly;
        memset(&ly, 0, sizeof ly);
        for (int e = 0; e < h.n; e++) {
            if (h.p_off[e + 1] == h.p_off[e]) continue;
            if (ly.n >= sh.maxe || h.down_fmt[e] != sh.down_fmt) {
                set_err("persistent decode: layer %d needs %d active experts with Q6_K down", l, sh.maxe);
                return false;
            }
            ly.gate[ly.n] = (const uint8_t *)(uintptr_t)h.gate[e];
            ly.up[ly.n] = (const uint8_t *)(uintptr_t)h.up[e];
            ly.down[ly.n] = (const uint8_t *)(uintptr_t)h.down[e];
            ly.w[ly.n] = h.p_w[h.p_off[e]];
            ly.n++;
        }
        if (ly.n != sh.maxe) {
            set_err("persistent decode: layer %d has %d active experts, the kernel runs exactly %d", l, ly.n,
                    sh.maxe);
            return false;
        }
        ly.norm_w = d->norm_w.empty() ? nullptr : d->norm_w[l];
        out.push_back(ly);
    }
    return true;
}

/* The multi-row kernel covers steps of k = 2..ROWS_MAXK rows of the Qwen
 * expert shape (up to ROWS_MAXE active experts and ROWS_MAXP pairs per
 * layer).  It builds the kernel's layer table and its buffers, each layer's
 * its own: tagged q8 rows of x [L][ROWS_MAXK][2 XS] | item ranges
 * [L][2][ROWS_GRID + 1] | the layers' expert and pair tables | tagged hidden
 * words [P_l][I] | tagged partials [P_l][D]. */
static bool persistent_rows_create(tg_hip_decode *d) {
    const DecodeShape sh = decode_qwen_shape();
    if (d->k < 2 || d->k > ROWS_MAXK) {
        set_err("persistent decode: the multi-row kernel runs 2 to %d rows, the plans hold %d", ROWS_MAXK, d->k);
        return false;
    }
    int pmax = 1;
    for (int l = 0; l < d->L; l++) {
        const HostPlan &h = d->plans[l]->h;
        if (h.D != sh.D || h.I != sh.I || h.gate_fmt != sh.gate_fmt || h.act != TG_ACT_SILU || h.has_gb || h.has_ub ||
            h.has_db) {
            set_err("persistent decode: layer %d is not a SiLU Q4_K gate/up step of %dx%d without biases", l, sh.D,
                    sh.I);
            return false;
        }
        int n_act = 0;
        for (int e = 0; e < h.n; e++)
            if (h.p_off[e + 1] > h.p_off[e]) {
                n_act++;
                if (h.down_fmt[e] != sh.down_fmt) {
                    set_err("persistent decode: layer %d has an active expert whose down matrix is not Q6_K", l);
                    return false;
                }
            }
        if (n_act > ROWS_MAXE || h.P > ROWS_MAXP) {
            set_err("persistent decode: layer %d has %d active experts and %d pairs; the multi-row kernel takes at "
                    "most %d and %d", l, n_act, h.P, ROWS_MAXE, ROWS_MAXP);
            return false;
        }
        pmax = std::max(pmax, h.P);
    }
    if (decode_rows_max_grid() < ROWS_GRID) {
        set_err("persistent decode: the multi-row kernel needs %d co-resident workgroups (co-resident %d)", ROWS_GRID,
                decode_rows_max_grid());
        return false;
    }
    const size_t XS = q8_lds_stride(sh.D / 256), NS = 2 * (ROWS_GRID + 1);
    size_t words = 0;   /* tagged hidden and partial words of all layers */
    for (int l = 0; l < d->L; l++) words += (size_t)d->plans[l]->h.P * (sh.I + sh.D);
    const size_t o_xq = 0, o_split = o_xq + (size_t)d->L * ROWS_MAXK * 2 * XS,
                 o_tab = (o_split + (size_t)d->L * NS * 4 + 255) & ~(size_t)255,
                 o_words = o_tab + (size_t)d->L * ROWS_TAB_BYTES, total = o_words + words * 8;
    HIPCHECK(hipMalloc(&d->hidden, total));
    HIPCHECK(hipMemset(d->hidden, 0, total));
    uint8_t *base = (uint8_t *)d->hidden;
    std::vector<int> splits((size_t)d->L * NS);
    std::vector<RowsLayer> ls(d->L);
    uint64_t *wp = (uint64_t *)(base + o_words);
    for (int l = 0; l < d->L; l++) {
        const tg_hip_moe_plan *p = d->plans[l];
        const HostPlan &h = p->h;
        std::vector<int> np;
        std::vector<uint8_t> tab(ROWS_TAB_BYTES, 0);
        for (int e = 0; e < h.n; e++) {
            if (h.p_off[e + 1] == h.p_off[e]) continue;
            RowsExp x = {h.gate[e], h.up[e], h.down[e], h.p_off[e], h.p_off[e + 1] - h.p_off[e]};
            memcpy(tab.data() + np.size() * sizeof x, &x, sizeof x);
            np.push_back(x.np);
        }
        const size_t n_act = np.size();
        memcpy(tab.data() + n_act * 32, h.p_row.data(), (size_t)h.P * 4);
        memcpy(tab.data() + n_act * 32 + (size_t)h.P * 4, h.p_w.data(), (size_t)h.P * 4);
        memcpy(tab.data() + n_act * 32 + (size_t)h.P * 8, h.r_off.data(), (size_t)(h.k + 1) * 4);
        memcpy(tab.data() + n_act * 32 + (size_t)h.P * 8 + (size_t)(h.k + 1) * 4, h.r_pair.data(), (size_t)h.P * 4);
        const size_t tb = (n_act * 32 + (size_t)h.P * 12 + (size_t)(h.k + 1) * 4 + 15) & ~(size_t)15;
        HIPCHECK(hipMemcpy(base + o_tab + (size_t)l * ROWS_TAB_BYTES, tab.data(), tb, hipMemcpyHostToDevice));
        decode_rows_split(np.data(), (int)n_act, d->k, splits.data() + (size_t)l * NS);
        RowsLayer &r = ls[l];
        memset(&r, 0, sizeof r);
        r.tab = base + o_tab + (size_t)l * ROWS_TAB_BYTES;
        r.tab_bytes = (int)tb;
        r.split = (const int *)(base + o_split) + (size_t)l * NS;
        r.norm_w = d->norm_w.empty() ? nullptr : d->norm_w[l];
        r.hidden = wp;
        r.part = wp + (size_t)h.P * sh.I;
        wp += (size_t)h.P * (sh.I + sh.D);
        r.xq = base + o_xq + (size_t)l * ROWS_MAXK * 2 * XS;
        r.n_act = (int)np.size();
        r.P = h.P;
        r.k = d->k;
        r.rec_bytes = (int)(((size_t)2 * d->k * sh.D + (size_t)pmax * sh.I) * 4);
    }
    d->rows_rec = (size_t)ls[0].rec_bytes;
    HIPCHECK(hipMemcpy(base + o_split, splits.data(), splits.size() * 4, hipMemcpyHostToDevice));
    HIPCHECK(hipMalloc(&d->layers_rows, ls.size() * sizeof(RowsLayer)));
    HIPCHECK(hipMemcpy(d->layers_rows, ls.data(), ls.size() * sizeof(RowsLayer), hipMemcpyHostToDevice));
    HIPCHECK(hipMalloc(&d->sync, 256));
    HIPCHECK(hipMemset(d->sync, 0, 256));
    HIPCHECK(hipMalloc(&d->place, DECODE_GRID * sizeof(unsigned)));
    HIPCHECK(hipMemset(d->place, 0xFF, DECODE_GRID * sizeof(unsigned)));
    d->grid = ROWS_GRID;
    d->pol = 1;   /* no intra-XCD exchange: nothing to check about placement */
    return true;
}

/* Per layer: RMSNorm of h fused with q8 of the result (into the plan's q8
 * rows), then the MoE kernels, which add into h.  A layer without pairs
 * leaves h as it is. */
static void decode_enqueue(tg_hip_decode *d, hipStream_t st) {
    for (int l = 0; l < d->L; l++) {
        tg_hip_moe_plan *p = d->plans[l];
        if (p->h.P == 0) continue;
        MoeArgs a = p->a;
        a.xin = d->x;
        a.xq.f = d->x;
        a.out = d->h;
        launch_rms_norm_q8(d->h, d->norm_w.empty() ? nullptr : d->norm_w[l], d->x, d->k, d->D, d->eps, a.xq, st);
        launch_moe(a, p->h.fmts_present.data(), (int)p->h.fmts_present.size(), st, nullptr, false);
    }
}

/* Mode 2: the persistent kernel as the one cooperative node of a graph,
 * built from the step's current arguments (debug, timing and slot policy
 * included; a setter that changes one marks the graph stale and the next run
 * rebuilds it).  Where the runtime refuses the node, cexec stays null and the
 * run falls back to hipLaunchCooperativeKernel. */
static void coop_graph_drop(tg_hip_decode *d) {
    if (d->cexec) HIPCHECK(hipDeviceSynchronize());   /* no launch of it may be pending */
    if (d->cexec) HIPCHECK(hipGraphExecDestroy(d->cexec));
    if (d->cgraph) HIPCHECK(hipGraphDestroy(d->cgraph));
    d->cexec = nullptr;
    d->cgraph = nullptr;
}

static void coop_graph_build(tg_hip_decode *d) {
    coop_graph_drop(d);
    d->cstale = false;
    const void *layers = d->kind == 2   ? (const void *)d->layers_rows
                         : d->kind == 1 ? (const void *)d->layers_mx
                                        : (const void *)d->layers;
    int L = d->L, pol = d->pol;
    float *h = d->h;
    void *slots = d->hidden;
    unsigned *sync = d->sync, *place = d->place;
    float eps = d->eps;
    uint8_t *debug = d->debug;
    uint64_t *times = d->times;
    /* both kernels take (layers, L, h, slots, abort/epoch, eps, debug, times,
     * place, pol); the node copies the values at creation */
    void *args[] = {(void *)&layers, (void *)&L,     (void *)&h,     (void *)&slots, (void *)&sync,
                    (void *)&eps,    (void *)&debug, (void *)&times, (void *)&place, (void *)&pol};
    hipKernelNodeParams kp;
    memset(&kp, 0, sizeof kp);
    kp.func = (void *)(d->kind == 2 ? decode_rows_fn() : d->kind == 1 ? decode_mx_fn() : decode_qwen_fn());
    kp.gridDim = dim3(d->grid);
    kp.blockDim = dim3(d->kind == 2 ? decode_rows_threads() : d->kind == 1 ? decode_mx_threads() : decode_threads());
    kp.sharedMemBytes = 0;
    kp.kernelParams = args;
    kp.extra = nullptr;
    hipGraphNode_t node;
    hipKernelNodeAttrValue v;
    memset(&v, 0, sizeof v);
    v.cooperative = 1;
    if (hipGraphCreate(&d->cgraph, 0) != hipSuccess || hipGraphAddKernelNode(&node, d->cgraph, nullptr, 0, &kp) != hipSuccess ||
        hipGraphKernelNodeSetAttribute(node, hipKernelNodeAttributeCooperative, &v) != hipSuccess ||
        hipGraphInstantiate(&d->cexec, d->cgraph, nullptr, nullptr, 0) != hipSuccess) {
        (void)hipGetLastError();
        if (d->cexec) (void)hipGraphExecDestroy(d->cexec);
        if (d->cgraph) (void)hipGraphDestroy(d->cgraph);
        d->cexec = nullptr;
        d->cgraph = nullptr;
    }
}

TG_API void tg_hip_decode_destroy(tg_hip_decode *d);

TG_API tg_hip_decode *tg_hip_decode_create(tg_hip_moe_plan *const *plans, int n_layers, const float *const *norm_w_dev,
                                           float eps, float *h_dev, int use_graph) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (n_layers <= 0 || !plans || !h_dev) {
        set_err("tg_hip_decode_create: bad arguments");
        return nullptr;
    }
    ensure_init();
    tg_hip_decode *d = new tg_hip_decode();
    d->L = n_layers;
    d->D = plans[0]->h.D;
    d->k = plans[0]->h.k;
    if (!rms_norm_fits(d->D)) {
        set_err("tg_hip_decode_create: D = %d is above the RMSNorm kernel's 16384", d->D);
        delete d;
        return nullptr;
    }
    for (int l = 0; l < n_layers; l++) {
        if (!plans[l] || plans[l]->h.D != d->D || plans[l]->h.k != d->k) {
            set_err("tg_hip_decode_create: layer %d has a different shape", l);
            delete d;
            return nullptr;
        }
        d->plans.push_back(plans[l]);
        if (norm_w_dev) d->norm_w.push_back(norm_w_dev[l]);
    }
    d->eps = eps;
    d->h = h_dev;
    if (use_graph < 0 || use_graph > 3) {
        set_err("tg_hip_decode_create: mode %d (0 kernels, 1 graph, 2 persistent, 3 persistent plain launch)",
                use_graph);
        delete d;
        return nullptr;
    }
    d->mode = use_graph;
    HIPCHECK(hipMalloc(&d->x, (size_t)d->k * d->D * 4));
    if (use_graph >= 2) {
        std::vector<DecodeLayer> ls;
        std::vector<DecodeLayerMx> lm;
        const HostPlan &h0 = d->plans[0]->h;
        if (d->k > 1) {   /* the multi-row kernel */
            d->kind = 2;
            if (!persistent_rows_create(d)) {
                tg_hip_decode_destroy(d);
                return nullptr;
            }
            if (d->mode == 2) coop_graph_build(d);
            return d;
        }
        d->kind = h0.gate_fmt == TG_FMT_MXFP4 && h0.D == DECODE_MX_D ? 1 : 0;
        if (d->kind == 1 ? !persistent_mx_ok(d, lm) : !persistent_ok(d, ls)) {
            HIPCHECK(hipFree(d->x));
            delete d;
            return nullptr;
        }
        int cus = 0;
        HIPCHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, g.dev));
        const int maxg = d->kind == 1 ? decode_mx_max_grid() : decode_qwen_max_grid();
        if (d->L > 64) {
            set_err("persistent decode: at most 64 layers per step");
            HIPCHECK(hipFree(d->x));
            delete d;
            return nullptr;
        }
        if (maxg < DECODE_GRID) {
            set_err("persistent decode: needs %d co-resident workgroups (CUs %d, co-resident %d)", DECODE_GRID, cus,
                    maxg);
            HIPCHECK(hipFree(d->x));
            delete d;
            return nullptr;
        }
        d->grid = DECODE_GRID;
        HIPCHECK(hipMalloc(&d->place, DECODE_GRID * sizeof(unsigned)));
        HIPCHECK(hipMemset(d->place, 0xFF, DECODE_GRID * sizeof(unsigned)));
        if (d->kind == 1) {
            /* the kernel reads each gate and up matrix in the wave-segment
             * layout: one rewritten copy per (layer, expert slot, matrix) */
            const size_t mb = decode_mx_seg_bytes();
            HIPCHECK(hipMalloc(&d->mxgu, lm.size() * DECODE_MX_E * 2 * mb));
            for (size_t l = 0; l < lm.size(); l++)
                for (int e = 0; e < DECODE_MX_E; e++) {
                    uint8_t *dg = d->mxgu + ((l * DECODE_MX_E + e) * 2) * mb, *du = dg + mb;
                    HIPCHECK(launch_mx_wave_segments(lm[l].gate[e], dg, g.st));
                    HIPCHECK(launch_mx_wave_segments(lm[l].up[e], du, g.st));
                    lm[l].gate[e] = dg;
                    lm[l].up[e] = du;
                }
            HIPCHECK(hipMalloc(&d->layers_mx, lm.size() * sizeof(DecodeLayerMx)));
            HIPCHECK(hipMemcpy(d->layers_mx, lm.data(), lm.size() * sizeof(DecodeLayerMx), hipMemcpyHostToDevice));
            HIPCHECK(hipStreamSynchronize(g.st));
        } else {
            /* the kernel reads each down matrix in the row-group layout: one
             * rewritten copy per (layer, expert slot) */
            const DecodeShape sh = decode_qwen_shape();
            const size_t mb = (size_t)sh.D * row_bytes(TG_FMT_Q6K, sh.I);
            HIPCHECK(hipMalloc(&d->qdown, ls.size() * DECODE_MAXE * mb));
            for (size_t l = 0; l < ls.size(); l++)
                for (int e = 0; e < DECODE_MAXE; e++) {
                    uint8_t *dst = d->qdown + (l * DECODE_MAXE + e) * mb;
                    HIPCHECK(launch_q6k_row_groups(ls[l].down[e], dst, sh.D, sh.I / 256, g.st));
                    ls[l].down[e] = dst;
                }
            HIPCHECK(hipMalloc(&d->layers, ls.size() * sizeof(DecodeLayer)));
            HIPCHECK(hipMemcpy(d->layers, ls.data(), ls.size() * sizeof(DecodeLayer), hipMemcpyHostToDevice));
            HIPCHECK(hipStreamSynchronize(g.st));
        }
        const size_t sb = d->kind == 1 ? decode_mx_slot_bytes() : decode_qwen_slot_bytes(d->grid);
        HIPCHECK(hipMalloc(&d->hidden, sb));   /* the exchange slots */
        HIPCHECK(hipMemset(d->hidden, 0, sb));
        HIPCHECK(hipMalloc(&d->sync, 256));
        HIPCHECK(hipMemset(d->sync, 0, 256));
        if (d->mode == 2) coop_graph_build(d);
        return d;
    }
    if (use_graph) {
        hipStream_t cs;
        HIPCHECK(hipStreamCreateWithFlags(&cs, hipStreamNonBlocking));
        HIPCHECK(hipStreamBeginCapture(cs, hipStreamCaptureModeThreadLocal));
        decode_enqueue(d, cs);
        HIPCHECK(hipStreamEndCapture(cs, &d->graph));
        HIPCHECK(hipGraphInstantiate(&d->exec, d->graph, nullptr, nullptr, 0));
        HIPCHECK(hipStreamDestroy(cs));
    }
    return d;
}

TG_API void tg_hip_decode_run(tg_hip_decode *d, void *stream) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!d) return;
    hipStream_t st = stream ? (hipStream_t)stream : g.st;
    if (d->mode == 2 && d->cstale) coop_graph_build(d);
    if (d->mode == 2 && d->cexec) {
        HIPCHECK(hipGraphLaunch(d->cexec, st));
    } else if (d->mode >= 2 && d->kind == 2) {
        HIPCHECK(launch_decode_rows(d->layers_rows, d->L, d->h, d->sync, d->eps, d->debug, d->times, d->place,
                                    d->mode == 2, st));
    } else if (d->mode >= 2 && d->kind == 1) {
        HIPCHECK(launch_decode_mx(d->layers_mx, d->L, d->h, d->hidden, d->sync, d->eps, d->debug, d->times, d->place,
                                  d->pol, d->mode == 2, st));
    } else if (d->mode >= 2) {
        HIPCHECK(launch_decode_qwen(d->layers, d->L, d->h, d->hidden, d->sync, d->eps, d->debug, d->times, d->place,
                                    d->pol, d->grid, d->mode == 2, st));
    } else if (d->exec) {
        HIPCHECK(hipGraphLaunch(d->exec, st));
    } else {
        decode_enqueue(d, st);
    }
    HIPCHECK(hipGetLastError());
}

/* Persistent steps write one debug record per layer into debug_dev
 * (tg_hip_decode_debug_bytes() each) while it is set; NULL turns it off. */
TG_API void tg_hip_decode_set_debug(tg_hip_decode *d, void *debug_dev) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!d) return;
    d->cstale |= d->debug != (uint8_t *)debug_dev;
    d->debug = (uint8_t *)debug_dev;
}

TG_API size_t tg_hip_decode_debug_bytes(void) { return (size_t)DecodeDebug::BYTES; }

/* Per-layer debug record bytes of this step's persistent kernel (the Qwen3
 * record above, or the gpt-oss record: h_in | x | hidden of each expert slot,
 * f32 of width 2880); 0 for a step that is not persistent. */
TG_API size_t tg_hip_decode_record_bytes(tg_hip_decode *d) {
    if (!d || d->mode < 2) return 0;
    if (d->kind == 2) return d->rows_rec;
    return d->kind == 1 ? (size_t)DecodeDebugMx::BYTES : (size_t)DecodeDebug::BYTES;
}

/* Persistent steps record up to 24 timing words per layer (timestamps of
 * the 100 MHz device clock, poll round counts) of every workgroup into
 * times_dev [256][L][24] (uint64) while it is set; NULL turns it off. */
TG_API void tg_hip_decode_set_timing(tg_hip_decode *d, void *times_dev) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!d) return;
    d->cstale |= d->times != (uint64_t *)times_dev;
    d->times = (uint64_t *)times_dev;
}

/* Persistent steps: true if, in the last launch, the workgroups g of each
 * class g % 8 all ran on one XCD -- what their intra-XCD exchanges need under
 * policy 0 (which XCD a class gets, and whether two classes share one, only
 * affects speed: a plain launch may start the round robin on another XCD). */
static bool placement_ok(tg_hip_decode *d) {
    if (!d->place) return true;
    unsigned x[DECODE_GRID];
    HIPCHECK(hipMemcpy(x, d->place, sizeof x, hipMemcpyDeviceToHost));
    for (int i = 8; i < DECODE_GRID; i++)
        if (x[i] != x[i % 8]) return false;
    return true;
}

/* 0 if every persistent step so far completed its exchange waits; 1 if a
 * wait timed out (the results of that step are invalid).  2 if a launch
 * split a class of workgroups g % 8 over several XCDs,
 * which its intra-XCD exchanges do not allow under policy 0: the step then
 * switches itself to storing every slot device-coherently
 * (tg_hip_decode_set_policy 1); the launches before the switch are suspect
 * (a wait that timed out among them also reports 1). */
TG_API int tg_hip_decode_status(tg_hip_decode *d) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!d || d->mode < 2) return 0;
    unsigned w;
    HIPCHECK(hipStreamSynchronize(g.st));
    HIPCHECK(hipMemcpy(&w, d->sync, 4, hipMemcpyDeviceToHost));
    if (w) return 1;
    if (d->pol == 0 && !placement_ok(d)) {
        d->placement_bad = 1;
        d->pol = 1;
        d->cstale = true;
    }
    return d->placement_bad ? 2 : 0;
}

/* Exchange-slot policy of the persistent steps: 0 keeps slots read only
 * inside one XCD in that XCD's L2 (needs workgroup g on XCD g % 8; the
 * default), 1 stores every slot device-coherently (correct under any
 * placement, slower).  Both give the same bits.  Returns the previous
 * policy, or -1 for a step that is not a persistent kernel. */
TG_API int tg_hip_decode_set_policy(tg_hip_decode *d, int pol) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!d || d->mode < 2) return -1;
    const int prev = d->pol;
    d->pol = pol ? 1 : 0;
    d->cstale |= d->pol != prev;
    return prev;
}

/* HW_REG_XCC_ID of each of the persistent step's 256 workgroups in its last
 * launch (out[256]); returns the number written (0 if none). */
TG_API int tg_hip_decode_placement(tg_hip_decode *d, unsigned *out) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!d || !d->place || !out) return 0;
    HIPCHECK(hipStreamSynchronize(g.st));
    HIPCHECK(hipMemcpy(out, d->place, DECODE_GRID * sizeof(unsigned), hipMemcpyDeviceToHost));
    return DECODE_GRID;
}

TG_API void tg_hip_decode_destroy(tg_hip_decode *d) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!d) return;
    HIPCHECK(hipStreamSynchronize(g.st));
    if (d->exec) HIPCHECK(hipGraphExecDestroy(d->exec));
    if (d->graph) HIPCHECK(hipGraphDestroy(d->graph));
    coop_graph_drop(d);
    HIPCHECK(hipFree(d->x));
    if (d->layers) HIPCHECK(hipFree(d->layers));
    if (d->layers_mx) HIPCHECK(hipFree(d->layers_mx));
    if (d->layers_rows) HIPCHECK(hipFree(d->layers_rows));
    if (d->hidden) HIPCHECK(hipFree(d->hidden));
    if (d->sync) HIPCHECK(hipFree(d->sync));
    if (d->qdown) HIPCHECK(hipFree(d->qdown));
    if (d->mxgu) HIPCHECK(hipFree(d->mxgu));
    if (d->place) HIPCHECK(hipFree(d->place));
    delete d;
}

/* Runs `iters` decode steps back to back on the library stream between two
 * HIP events and returns the elapsed milliseconds. */
TG_API float tg_hip_decode_time(tg_hip_decode *d, int iters) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!d || iters <= 0) return 0.f;
    hipEvent_t a, b;
    HIPCHECK(hipEventCreate(&a));
    HIPCHECK(hipEventCreate(&b));
    HIPCHECK(hipEventRecord(a, g.st));
    for (int i = 0; i < iters; i++) tg_hip_decode_run(d, nullptr);
    HIPCHECK(hipEventRecord(b, g.st));
    HIPCHECK(hipEventSynchronize(b));
    float ms = 0.f;
    HIPCHECK(hipEventElapsedTime(&ms, a, b));
    HIPCHECK(hipEventDestroy(a));
    HIPCHECK(hipEventDestroy(b));
    return ms;
}

/* One eager decode step with HIP events around every kernel; returns the
 * summed milliseconds per kernel class in ms_out[6] = {rms_norm,
 * quantize(x), gate/up, quantize(hidden), down, combine} and their launch
 * counts in n_out[6]. */
TG_API void tg_hip_decode_kernel_times(tg_hip_decode *d, float *ms_out, int *n_out) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!d) return;
    for (int i = 0; i < 6; i++) {
        ms_out[i] = 0.f;
        n_out[i] = 0;
    }
    if (d->mode >= 2) return;   /* one kernel per step: tg_hip_decode_time is its duration */
    std::vector<hipEvent_t> ev;
    std::vector<int> cls;
    auto mark = [&](int c) {
        hipEvent_t e;
        HIPCHECK(hipEventCreate(&e));
        HIPCHECK(hipEventRecord(e, g.st));
        ev.push_back(e);
        cls.push_back(c);
    };
    for (int l = 0; l < d->L; l++) {
        tg_hip_moe_plan *p = d->plans[l];
        if (p->h.P == 0) continue;
        MoeArgs a = p->a;
        a.xin = d->x;
        a.xq.f = d->x;
        a.out = d->h;
        mark(-1);
        launch_rms_norm_q8(d->h, d->norm_w.empty() ? nullptr : d->norm_w[l], d->x, d->k, d->D, d->eps, a.xq, g.st);
        mark(0);
        std::function<void(int)> mk = [&](int c) { mark(c); };
        launch_moe(a, p->h.fmts_present.data(), (int)p->h.fmts_present.size(), g.st, &mk, false);
    }
    HIPCHECK(hipStreamSynchronize(g.st));
    for (size_t i = 1; i < ev.size(); i++) {
        if (cls[i] < 0) continue;
        float ms;
        HIPCHECK(hipEventElapsedTime(&ms, ev[i - 1], ev[i]));
        ms_out[cls[i]] += ms;
        n_out[cls[i]] += 1;
    }
    for (auto e : ev) HIPCHECK(hipEventDestroy(e));
}

TG_API void tg_hip_device_name(char *buf, int n) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    ensure_init();
    hipDeviceProp_t pr;
    HIPCHECK(hipGetDeviceProperties(&pr, g.dev));
    snprintf(buf, (size_t)n, "%s (%s, %d CUs)", pr.name, pr.gcnArchName, pr.multiProcessorCount);
}

/* Pairs per expert from which MXFP4 expert layers take the int8 MFMA phases
 * (0: never); returns the previous setting. */
TG_API int tg_hip_set_moe_grouped_min_rows(int rows) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    const int prev = grouped_min_rows();
    set_grouped_min_rows(rows);
    return prev;
}

/* Pairs per expert from which Q4_K gate/up + Q6_K down expert layers take
 * the int8 MFMA phases (0: never; negative: the default by shape); returns
 * the previous setting. */
TG_API int tg_hip_set_moe_qk_min_rows(int rows) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    const int prev = qk_min_rows();
    set_qk_min_rows(rows);
    return prev;
}

/* Input-row count from which the fused q6_K head runs on int8 MFMA (0:
 * never); returns the previous setting. */
TG_API int tg_hip_set_head_mfma_min_k(int k) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    return set_head_mfma_min_k(k);
}

/* Q4_K / Q6_K expert layers: expert-major phases (mode bits, default 7) or
 * one workgroup column per pair (0); the same bits either way.  Returns the
 * previous mode. */
TG_API int tg_hip_set_moe_expert_major(int mode) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    const int prev = expert_major();
    set_expert_major(mode < 0 ? EM_DEFAULT : mode);
    return prev;
}

/* Event marks on the library stream, for timing queued device work. */
static hipEvent_t g_marks[8];
static bool g_marks_ready = false;

static void release_marks() {
    if (!g_marks_ready) return;
    for (auto &e : g_marks) HIPCHECK(hipEventDestroy(e));
    g_marks_ready = false;
}

TG_API void tg_hip_mark(int slot) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    ensure_init();
    if (slot < 0 || slot >= 8) {
        set_err("tg_hip_mark: slot must be 0..7");
        return;
    }
    if (!g_marks_ready) {
        for (auto &e : g_marks) HIPCHECK(hipEventCreate(&e));
        g_marks_ready = true;
    }
    HIPCHECK(hipEventRecord(g_marks[slot], g.st));
}

TG_API float tg_hip_marks_ms(int a, int b) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!g_marks_ready || a < 0 || a >= 8 || b < 0 || b >= 8) {
        set_err("tg_hip_marks_ms: record both marks first");
        return 0.f;
    }
    HIPCHECK(hipEventSynchronize(g_marks[b]));
    float ms = 0.f;
    HIPCHECK(hipEventElapsedTime(&ms, g_marks[a], g_marks[b]));
    return ms;
}

/* Copies nbytes (multiple of 16) device-to-device with a plain vector-load
 * kernel `iters` times on the library stream; returns ms (HIP events).  The
 * reference point for measured HBM bandwidth and for counter calibration. */
TG_API float tg_hip_copy_time(const void *src_dev, void *dst_dev, uint64_t nbytes, int iters) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    ensure_init();
    if (nbytes % 16 || iters <= 0) {
        set_err("tg_hip_copy_time: nbytes must be a multiple of 16");
        return 0.f;
    }
    hipEvent_t a, b;
    HIPCHECK(hipEventCreate(&a));
    HIPCHECK(hipEventCreate(&b));
    HIPCHECK(hipEventRecord(a, g.st));
    for (int i = 0; i < iters; i++) launch_copy(src_dev, dst_dev, nbytes, g.st);
    HIPCHECK(hipEventRecord(b, g.st));
    HIPCHECK(hipEventSynchronize(b));
    float ms = 0.f;
    HIPCHECK(hipEventElapsedTime(&ms, a, b));
    HIPCHECK(hipEventDestroy(a));
    HIPCHECK(hipEventDestroy(b));
    return ms;
}
