/*
 * tg_kernels.h -- launch interface between the C-ABI layer (tg_api.hip) and
 * the kernels (tg_kernels.hip).  Internal to libtinygiant_hip.
 */
#ifndef TG_KERNELS_H
#define TG_KERNELS_H
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <functional>
#include <vector>

#include "tg_common.h"
#include "tg_device.hpp"

namespace tg {

/* One active expert of a layer call, read by a workgroup of the
 * expert-major phases in one scalar burst: weight addresses, its pairs
 * [p0, p0 + np) and the input rows of the first EXP_ROWS of them. */
#define EXP_ROWS 8
struct ExpDesc {
    uint64_t gate, up, down;
    int e, p0, np, down_fmt;
    int row[EXP_ROWS];
};

/* Everything one MoE layer call needs, all pointers on the device.
 * Pairs p = (expert e, active input row) are numbered expert-major, in the
 * order the reference gathers them (csrc/libtinygiant.c:1411-1423). */
struct MoeArgs {
    const uint64_t *gate, *up, *down;       /* [n] weight base addresses */
    const int *down_fmt;                    /* [n] */
    const uint64_t *gbias, *ubias, *dbias;  /* [n] or null; entries may be 0 */
    const int *p_off;                       /* [n+1] first pair of each expert */
    const int *p_row;                       /* [P] input row of the pair */
    const int *p_exp;                       /* [P] expert of the pair */
    const float *p_w;                       /* [P] router weight of the pair */
    const int *r_off;                       /* [k+1] first entry of each output row */
    const int *r_pair;                      /* [P] pairs of each output row, expert order */
    const float *xin;                       /* [k][D] inputs */
    Q8Rows xq;                              /* [k] quantized inputs */
    float *hidden;                          /* [P][I] */
    Q8Rows hq;                              /* [P] quantized hidden */
    float *part;                            /* [P][D] weighted down outputs */
    float *out;                             /* [k][D] accumulated output */
    int n, k, P, D, I, act, gate_fmt;
    uint32_t gate_rb;
    int max_rows;                           /* most pairs of any one expert */
    int mx_aligned;                         /* every MXFP4 matrix of an active expert starts 16-byte aligned */
    int mx_e255;                            /* an active MXFP4 matrix holds an e8m0 scale byte of 255 */
    const int *mx_act;                      /* active experts, then active experts with an MXFP4 down matrix */
    const int *mx_cum;                      /* cost prefix of each list (n_act + 1 entries each) */
    uint8_t *xp, *hp;                       /* fp8 halves of xq / hq rows in MFMA order, or null */
    int n_act_a, n_act_b;
    const ExpDesc *ed;                      /* [n_act_a] active experts, the most pairs first */
    unsigned *ctr;                          /* [ctr_n] row-tile tickets of the fused combine, zero between calls, or null */
    int ctr_n;
    int xin_remote;                         /* xin lies in host memory: quantize it once, in its own launch */
    const int *rg_items, *rg_off;           /* the persistent gate/up phase's items and each workgroup's range, or null */
    const int *rg_rend;                     /* for each item, the end of its run (items of one expert and pass) */
    const int *rg_runs, *rg_run0;           /* each run's record (RING_REC ints) and each workgroup's first run */
    int rg_n;                               /* its workgroups */
    const int *rb_items, *rb_off, *rb_rend; /* the persistent down phase's, or null */
    const int *rb_runs, *rb_run0;
    int rb_n;
};

int items_per_row(int fmt, int ncols);
uint32_t row_bytes(int fmt, int ncols);

/* q8 of nrows rows; clear[0 .. nclear) (nclear <= 64) are zeroed on the way,
 * for a consumer launched next (the fused head's argmax keys) */
void launch_quantize(const float *x, int ncols, int nrows, long xstride, const Q8Rows &out, hipStream_t st,
                     unsigned long long *clear = nullptr, int nclear = 0);
void launch_gemv(int fmt, const uint8_t *W, int nrows, int ncols, const float *bias, const Q8Rows &x, int k,
                 float *y, long ystride, hipStream_t st);
/* up to three matrices of one format and width (ncols) against the same q8
 * rows, one launch: y_j[r] = dot(W_j row r, x) + bias_j[r] */
struct GemvJob {
    const uint8_t *W;
    const float *bias;
    float *y;
    long ystride;
    int nrows;
};
struct GemvJobs {
    GemvJob j[3];
};
void launch_gemv_multi(int fmt, const GemvJobs &jobs, int njobs, int ncols, const Q8Rows &x, int k, hipStream_t st);
/* q8 of one f32 row (ncols % 256 == 0, at most Q8X_MAX_BLOCKS blocks) and
 * up to three Q4_K / Q6_K GEMVs of it in one launch (fmts[j] per job); the
 * same bits as launch_quantize + launch_gemv_multi.  Also clears n_zero
 * (<= 256) words at `zero` with device-scope stores. */
#define Q8X_MAX_BLOCKS 32
struct GemvQ8xMap {
    int wg0[4];     /* first workgroup of each job, then the total */
    int fmt[3];
    uint32_t rb[3];
};
bool gemv_q8x_ok(const int *fmts, int njobs, int ncols);
void launch_gemv_q8x(const int *fmts, const GemvJobs &jobs, int njobs, int ncols, const float *x, unsigned *zero,
                     int n_zero, hipStream_t st);
void launch_isums(int fmt, const uint8_t *W, int nrows, int ncols, const Q8Rows &x, int nsums_row, int32_t *out,
                  hipStream_t st);
/* `mark`, when given, is called after each kernel with its class:
 * 1 quantize(x), 2 gate/up, 3 quantize(hidden), 4 down, 5 combine.
 * quantize_x false: a.xq already holds q8 of the input rows. */
void launch_moe(const MoeArgs &a, const int *down_fmts_present, int n_down_fmts, hipStream_t st,
                const std::function<void(int)> *mark = nullptr, bool quantize_x = true);
/* MXFP4 phases on block-scaled MFMA with LDS-resident weight slabs
 * (tg_grouped.hip): every weight byte is read once whatever the pairs per
 * expert.  launch_mx_split prepares the fp8 halves of q8 rows. */
bool grouped_lds_ok(int D, int I);
void launch_mx_split(const Q8Rows &q, int nrows, int ncols, uint8_t *dst, hipStream_t st);
/* sets *flag_dev (not cleared here) when a block of the MXFP4 bytes at p
 * (nbytes, whole 17-byte blocks) has the scale byte 255 */
void launch_mx_scan_e255(const uint8_t *p, uint64_t nbytes, unsigned *flag_dev, hipStream_t st);
void launch_moe_a_mx(const MoeArgs &a, hipStream_t st);
void launch_moe_b_mx(const MoeArgs &a, hipStream_t st);
/* pairs per expert from which launch_moe takes the MFMA phases for MXFP4
 * experts; 0 switches them off */
void set_grouped_min_rows(int rows);
int grouped_min_rows();
/* Q4_K gate/up and Q6_K down phases on int8 MFMA with LDS-resident weight
 * slabs (tg_grouped_k.hip), taken by launch_moe for layers whose experts
 * hold at least qk_min_rows() pairs (0: never; negative: the default by
 * shape, 17 where both persistent rings run, 40 elsewhere) */
bool qk_grouped_fits(const MoeArgs &a);
/* The persistent int8 MFMA gate/up phase (Q4_K, D = 2048): its items, (index
 * ei into the busiest-first active experts, 16-row slab s, pass t of 16
 * pairs) as ei << 16 | s << 8 | t, and off[0 .. G] the range of each of G
 * workgroups.  False when the shape is not the phase's. */
bool qa_ring_shape(int gate_fmt, int D, int I);
bool qb_ring_shape(int I, int D);
/* The persistent phases' items (expert, pass, slab of `slabs`) cut into G
 * workgroup ranges (off), the end of each item's run (rend: the items of one
 * expert and pass), the runs' records (RING_REC ints each: the run's first
 * pair p0 + 16 t, the pairs from there on, np - 16 t, possibly more than 16,
 * and the input rows of its first 16 pairs, the last pair's row past the
 * end) and the run of each workgroup's first item (run0). */
constexpr int RING_REC = 20;
struct RingLists {
    std::vector<int> items, off, rend, runs, run0;
};
void ring_items(const ExpDesc *ed, int n_act, int slabs, int G, const int *p_row, int P, RingLists &r);
constexpr int QA_RING_MAX_G = 1024;
void launch_moe_a_qk(const MoeArgs &a, hipStream_t st);
void launch_moe_b_qk(const MoeArgs &a, hipStream_t st);
void set_qk_min_rows(int rows);
int qk_min_rows();
/* Q4_K / Q6_K experts: one workgroup column per active expert, each weight
 * row read once for all its pairs (EM_ON), or one per pair (0).  For layers
 * with at most two pairs per expert: EM_FUSE_Q8, the phases quantize their
 * rows themselves; EM_TICKETS, the down phase also combines (row-tile
 * tickets).  EM_FUSE_ANY: those two whatever the pair count (for tests). */
enum { EM_ON = 1, EM_FUSE_Q8 = 2, EM_TICKETS = 4, EM_FUSE_ANY = 8, EM_DEFAULT = 7, EM_ALL = 15 };
void set_expert_major(int mode);
int expert_major();
/* RMSNorm rows of n <= 16384 values (rms_norm_fits); the _q8 form also
 * writes q8 of the result to q, bit-identical to launch_quantize over it */
bool rms_norm_fits(int n);
void launch_rms_norm(const float *x, const float *w, float *out, int nrows, int n, float eps, hipStream_t st);
void launch_rms_norm_q8(const float *x, const float *w, float *out, int nrows, int n, float eps, const Q8Rows &q,
                        hipStream_t st, unsigned long long *clear = nullptr, int nclear = 0);
void launch_synth_fill(int kind, uint64_t seed, void *dst, uint64_t nbytes, hipStream_t st);
void launch_copy(const void *src, void *dst, uint64_t nbytes, hipStream_t st);

}  // namespace tg
#endif
