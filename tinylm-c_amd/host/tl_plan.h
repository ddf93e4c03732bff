/* tl_plan.h -- the GEMM call sequences of tinylm.c as data, and their device
 * executor (libtlhost.so, plain C over the libtlgemm C ABI).
 *
 * A plan is the ordered list of mm / mm_bt / mm_atb calls (plus the memsets
 * that set an accumulation base) that the reference issues for one training
 * step or one decode token, with each operand named by a buffer of the
 * reference (tinylm.c's Acts fields, the flat parameter buffer P and grad
 * buffer G with map_weights' offsets, tinylm.c:361-393) and the tinylm.c line
 * of the call.  The executor keeps every buffer resident in HBM and issues the
 * calls on one stream, so host <-> device copies happen only at step
 * boundaries.
 */
#ifndef TL_PLAN_H
#define TL_PLAN_H
#include <stddef.h>
#ifdef __cplusplus
extern "C" {
#endif

enum { TL_MM = 0, TL_MM_BT = 1, TL_MM_ATB = 2, TL_ZERO = 3 };

/* How the bench / tests initialise a buffer (BASELINE inputs). */
enum { TL_INIT_ACT = 0,     /* X  ~ N(0, 1)          activations            */
       TL_INIT_WEIGHT = 1,  /* W  ~ N(0, 0.02^2)     parameters             */
       TL_INIT_GRAD = 2,    /* dY ~ N(0, 0.01^2)     upstream gradients     */
       TL_INIT_ZERO = 3 };  /* accumulators (G, outputs)                     */

#define TL_MAXBUF 48
#define TL_NAMELEN 16

typedef struct {
    char name[TL_NAMELEN];
    size_t floats;
    int init;
} TlBuf;

typedef struct {
    int op;                 /* TL_MM, TL_MM_BT, TL_MM_ATB, TL_ZERO          */
    int out, a, b;          /* buffer ids; a = b = -1 for TL_ZERO           */
    size_t out_off, a_off, b_off;   /* float offsets inside those buffers   */
    int M, K, N;            /* the reference call's own arguments           */
    size_t n;               /* TL_ZERO: floats cleared                      */
    int line;               /* tinylm.c line of the call                    */
    char what[TL_NAMELEN];  /* short label, e.g. "q", "dW2", "logits"       */
    int run;                /* GEMM run: calls with the same run index are
                               issued back to back by the reference with no
                               non-GEMM code between them                   */
    int hoist;              /* TL_ZERO only: nothing the reference runs
                               between the previous GEMM run and this clear
                               reads or writes the cleared range, so the
                               clear may run with that run's launch         */
} TlCall;

typedef struct {
    int nbuf, ncall, cap;
    TlBuf buf[TL_MAXBUF];
    TlCall *call;
    /* model shape the plan was built for */
    int R, D, KD, F, V, L, n_mtp;
    int run;                /* current run index while building */
} TlPlan;

/* Offsets of one layer's weights inside the flat P/G buffer
 * (map_weights, tinylm.c:361-393, dense FFN, no QK-norm). */
typedef struct { size_t emb, an1, wq, wk, wv, wo, an2, w1, w3, w2, nf, mtp0; size_t total; } TlWeightMap;
void tl_weight_map(int V, int D, int KD, int F, int L, int n_mtp, int layer, TlWeightMap *m);

/* One training step's GEMMs (forward tinylm.c:968-1029, mtp_grad :1036-1069,
 * backward :1072-1154) for R = B*T rows, plus the memset(G) of :2628.
 * Returns 0, or -1 on bad arguments / allocation failure. */
int  tl_plan_train(TlPlan *p, int R, int D, int KD, int F, int V, int L, int n_mtp);
/* One decode step's fp32 GEMMs for M rows (forward_chunk, tinylm.c:3721-3830,
 * with no int8 copy: mm_dec -> mm, mmbt_dec -> memset + mm_bt, :3029-3036). */
int  tl_plan_decode(TlPlan *p, int M, int D, int KD, int F, int V, int L);
/* The same GEMVs on the decode layout (tldecode.h tlg_dev_transpose: each
 * linear weight stored transposed at its map_weights offset): every
 * mm(M, K, N) becomes memset + mm_bt(M, N, K), so each GEMV streams whole
 * contiguous weight rows. */
int  tl_plan_decode_packed(TlPlan *p, int M, int D, int KD, int F, int V, int L);
void tl_plan_free(TlPlan *p);
int  tl_plan_find(const TlPlan *p, const char *name);
/* Algorithmic flops of call i (2*M*K*N for a GEMM, 0 for a clear) and the
 * compulsory bytes it moves (operands read once, output written once, plus
 * the output read for the accumulating forms). */
double tl_call_flops(const TlCall *c);
double tl_call_bytes(const TlCall *c);

/* ---- device executor ----------------------------------------------------- */
typedef struct TlRun TlRun;
/* Allocate every plan buffer in HBM (one arena).  `pool` > 1 allocates that
 * many copies of the parameter buffer P and rotates through them one step at
 * a time, so weights stream from HBM rather than the last-level cache. */
TlRun *tl_run_new(const TlPlan *p, int pool);
void   tl_run_free(TlRun *r);
/* Fill every buffer per its TlBuf.init with seeded Gaussians (on device). */
int    tl_run_fill(TlRun *r, unsigned long long seed, void *stream);
/* Device address of buffer `id` (pool copy 0 for P). */
float *tl_run_buf(TlRun *r, int id);
/* Enqueue one step (all calls in order) on `stream`. */
int    tl_run_step(TlRun *r, void *stream);
/* Enqueue call i only (for per-call timing). */
int    tl_run_call(TlRun *r, int i, void *stream);
/* Enqueue one step with each GEMM run as one grouped launch
 * (tlg_dev_gemm_group): a memset followed by an accumulating GEMM into the
 * same range becomes a setting GEMM, consecutive mm_bt into one dX become a
 * chain.  Same results up to fp32 rounding (and the sign of exact zeros). */
int    tl_run_step_grouped(TlRun *r, void *stream);
/* Number of kernel launches a grouped step issues (for reports), not
 * counting the final flush of split partials. */
int    tl_run_grouped_launches(TlRun *r);
/* One grouped step with events[k] recorded on `stream` before launch k and
 * events[L+1] after the flush (L = tl_run_grouped_launches; nevents >= L+2).
 * tl_run_launch_info then gives launch k's kind (0 grouped GEMMs, 1 clear,
 * 2 flush) and its algorithmic flops and compulsory bytes. */
int    tl_run_time_launches(TlRun *r, void **events, int nevents, void *stream);
int    tl_run_launch_info(TlRun *r, int k, double *flops, double *bytes);
/* Kernel that launch k of the last timed step ran, as rocprofv3 names it
 * (without "void " and the argument list), or NULL if nothing launched. */
const char *tl_run_launch_kernel(TlRun *r, int k);
/* Choose each grouped launch's tile configuration by timing: `reps` steps per
 * candidate (indices of the library's tile table, see tlg_tune_group), each
 * launch keeping its fastest.  Later grouped steps and graphs use the choice;
 * tl_run_launch_config reports it (-1 = the library's automatic policy). */
int    tl_run_autotune(TlRun *r, const int *cands, int ncands, int reps, void *stream);
int    tl_run_launch_config(TlRun *r, int k);
/* Pin launch k's tile configuration (an index of the library's tile table,
 * -1 = the automatic policy): a tuned table applied without re-timing. */
int    tl_run_set_launch_config(TlRun *r, int k, int cfg);
/* The same with split targets as well: every (cands[c], rts[s]) pair is
 * timed (rts: target reduction steps per split work item, tlg_tune_group_split
 * values; 0 = the library's automatic target), each launch keeping its
 * fastest pair; tl_run_autotune is this with rts = {0}.  tl_run_launch_split
 * reports launch k's target, tl_run_set_launch_split pins it. */
int    tl_run_autotune_split(TlRun *r, const int *cands, int ncands, const int *rts, int nrts, int reps,
                             void *stream);
int    tl_run_launch_split(TlRun *r, int k);
int    tl_run_set_launch_split(TlRun *r, int k, int rtarget);
/* Capture one step into a HIP graph and replay it (grouped != 0: the grouped
 * step, else call by call).  The graph is bound to
 * the pool copy current at capture; tl_run_graph_step replays the graph for
 * that copy (one graph per pool copy). */
int    tl_run_graph_build(TlRun *r, void *stream, int grouped);
int    tl_run_graph_step(TlRun *r, void *stream);

#ifdef __cplusplus
}
#endif
#endif
