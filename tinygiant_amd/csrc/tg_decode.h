/*
 * tg_decode.h -- the persistent decode-step kernel's interface (internal).
 */
#ifndef TG_DECODE_H
#define TG_DECODE_H
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tg {

constexpr int DECODE_MAXE = 8;    /* the persistent step runs exactly 8 experts per layer */
constexpr int DECODE_GRID = 256;   /* ... on 256 co-resident workgroups (one per MI355X CU) */

/* One layer of the step: its active experts (device pointers), their router
 * weights and the RMSNorm weight applied to h before the layer (null = 1). */
struct DecodeLayer {
    const uint8_t *gate[DECODE_MAXE];
    const uint8_t *up[DECODE_MAXE];
    const uint8_t *down[DECODE_MAXE];
    float w[DECODE_MAXE];
    const float *norm_w;
    int n;
};

/* Per-layer debug record written when a debug buffer is set (stage-wise
 * parity of the persistent step; h and x parts by workgroup 0, expert slot
 * e's hidden parts by the workgroup that owns expert e): byte offsets for D = 2048,
 * I = 768.  h_in f32[D] | x f32[D] | xq i8[D] | xd f32[D/256] | xs32 i32[D/32] |
 * hidden f32[8][I] | hq i8[8][I] | hd f32[8][I/256] | hs16 i32[8][I/16] */
struct DecodeDebug {
    static constexpr int D = 2048, I = 768, E = DECODE_MAXE;
    static constexpr int HIN = 0, X = HIN + D * 4, XQ = X + D * 4, XD = XQ + D, XS32 = XD + (D / 256) * 4,
                         HID = XS32 + (D / 32) * 4, HQ = HID + E * I * 4, HD = HQ + E * I,
                         HS16 = HD + E * (I / 256) * 4, BYTES = HS16 + E * (I / 16) * 4;
};

/* The gpt-oss-120b step (tg_decode_mx.hip): D = I = 2880, exactly 4 MXFP4
 * experts per layer with optional gate/up/down biases (f32 device vectors)
 * and the clamped SwiGLU. */
constexpr int DECODE_MX_E = 4;
constexpr int DECODE_MX_D = 2880;
struct DecodeLayerMx {
    const uint8_t *gate[DECODE_MX_E];
    const uint8_t *up[DECODE_MX_E];
    const uint8_t *down[DECODE_MX_E];
    const float *gb[DECODE_MX_E];
    const float *ub[DECODE_MX_E];
    const float *db[DECODE_MX_E];
    float w[DECODE_MX_E];
    const float *norm_w;
    int n, pad;
};
/* Its per-layer debug record: h_in f32[D] | x f32[D] | q8(x) quants i8[NQ*256]
 * (zero padded) | q8(x) scales f32[NQ] (workgroup 0) | hidden f32[4][D] |
 * q8(hidden) quants i8[4][NQ*256] | q8(hidden) scales f32[4][NQ] (expert
 * slot e's by workgroup 2e); NQ = 12 q8 blocks of 256 per row */
struct DecodeDebugMx {
    static constexpr int D = DECODE_MX_D, E = DECODE_MX_E, NQ = (DECODE_MX_D + 255) / 256;
    static constexpr int HIN = 0, X = HIN + D * 4, XQ = X + D * 4, XD = XQ + NQ * 256, HID = XD + NQ * 4,
                         HQ = HID + E * D * 4, HD = HQ + E * NQ * 256, BYTES = HD + E * NQ * 4;
};
int decode_mx_max_grid();
size_t decode_mx_slot_bytes();
hipError_t launch_decode_mx(const DecodeLayerMx *layers_dev, int L, float *h_dev, void *slots_dev, unsigned *abort_dev,
                            float eps, uint8_t *debug_dev, uint64_t *times_dev, unsigned *place_dev, int pol,
                            bool cooperative, hipStream_t st);
/* the persistent kernels' entry points and block size, for graph nodes */
const void *decode_mx_fn();
int decode_mx_threads();
const void *decode_qwen_fn();
int decode_threads();

/* Shape the persistent kernel is built for; the host checks a step against it. */
struct DecodeShape {
    int D, I, gate_fmt, down_fmt, maxe, threads;
};
DecodeShape decode_qwen_shape();

/* Queues one step.  slots_dev holds decode_qwen_slot_bytes(grid) zeroed
 * bytes; `base` advances by 2 * L per launch (slot tags are base-relative);
 * abort_dev is one word, nonzero after a timed-out wait.  A cooperative
 * launch fails unless every workgroup can be resident at once; a plain launch
 * relies on the device being otherwise idle (the occupancy check at set-up
 * shows one workgroup fits per CU), and a workgroup that never starts only
 * makes the others' bounded waits time out.  Returns the launch status. */
size_t decode_qwen_slot_bytes(int grid);
/* place_dev (grid words, or null) receives each workgroup's HW_REG_XCC_ID;
 * pol = 1 stores every exchange slot device-coherently (correct under any
 * placement), pol = 0 keeps intra-XCD slots in the writer's L2 (needs
 * workgroup g on XCD g % 8).  The down matrices of layers_dev are in the
 * row-group layout of launch_q6k_row_groups. */
hipError_t launch_decode_qwen(const DecodeLayer *layers_dev, int L, float *h_dev, void *slots_dev,
                              unsigned *abort_dev, float eps, uint8_t *debug_dev, uint64_t *times_dev,
                              unsigned *place_dev, int pol, int grid, bool cooperative, hipStream_t st);
int decode_qwen_max_grid();
/* Q6_K matrix (nrows x nb blocks, nrows % 8 == 0) -> row-group layout:
 * per 8 rows {ql[8 nb][128] | qh[8 nb][64] | sc[8 nb][16] | d[8 nb]}. */
hipError_t launch_q6k_row_groups(const void *src, void *dst, int nrows, int nb, hipStream_t st);

/* The multi-row step (tg_decode_rows.hip): k = 2..ROWS_MAXK rows of the
 * Qwen3 expert shape on ROWS_GRID co-resident workgroups.  One layer: its
 * active experts and pairs (a compact table the kernel stages in LDS), the
 * plan's per-row pair lists, the layer's own exchange buffers, and the
 * workgroups' item ranges: split[w] .. split[w + 1] of the gate/up items
 * (expert-major, 16 rows each) and split[ROWS_GRID + 1 + w] .. of the down
 * items (64 rows each).  Hidden values, partials and the 4-byte units of x
 * are 8-byte words {tag, value}; the tag of layer l in a launch is epoch +
 * l + 1. */
constexpr int ROWS_MAXK = 16;
constexpr int ROWS_GRID = 256;
constexpr int ROWS_MAXE = 128;    /* active experts of a layer */
constexpr int ROWS_MAXP = 256;    /* pairs of a layer */
/* an active expert: its matrices and its pairs [p0, p0 + np) */
struct RowsExp {
    uint64_t gate, up, down;
    int p0, np;
};
/* the layer's table: RowsExp [n_act] | pair rows int [P] | pair weights f32 [P]
 * | first entry of each row's pair list int [k + 1] | the lists int [P] */
constexpr int ROWS_TAB_BYTES = ROWS_MAXE * 32 + ROWS_MAXP * 12 + (ROWS_MAXK + 1) * 4 + 12;
struct RowsLayer {
    const uint8_t *tab;           /* the table above, tab_bytes (a multiple of 16) */
    const int *split;
    const float *norm_w;          /* RMSNorm weight before this layer, null = 1 */
    uint64_t *hidden, *part;      /* [P][I], [P][D] tagged words */
    uint8_t *xq;                  /* [k] q8 rows of x, the LDS image as tagged 4-byte units (2 XS bytes a row) */
    int n_act, P, k, rec_bytes;   /* rec_bytes: debug record of a layer */
    int tab_bytes, pad;
};
static_assert(sizeof(RowsExp) == 32, "table layout");
/* Per-layer debug record: h_in f32[k][D] | x f32[k][D] | hidden f32[Pmax][I] */
int decode_rows_max_grid();
/* the item ranges of one layer from each active expert's pair count; the
 * down items go to workgroups c .. ROWS_GRID - 1 (c: the rows combined) */
void decode_rows_split(const int *np, int n_act, int c, int *split /* [2 (ROWS_GRID + 1)] */);
hipError_t launch_decode_rows(const RowsLayer *layers_dev, int L, float *h_dev, unsigned *sync_dev, float eps,
                              uint8_t *debug_dev, uint64_t *times_dev, unsigned *place_dev, bool cooperative,
                              hipStream_t st);
const void *decode_rows_fn();
int decode_rows_threads();

}  // namespace tg
#endif
