/* tl_train.h -- a device-resident training step of tinylm.c (libtlhost.so,
 * plain C over the libtlgemm C ABI: include/tlgemm.h and include/tltrain.h).
 *
 * One TlTrain holds a model's flat parameter, gradient and AdamW moment
 * buffers (map_weights' layout, tinylm.c:361-393) and every activation the
 * backward pass reads (Acts, tinylm.c:654-696) in HBM.  A step is the
 * reference's train_loop body (:2627-2633): forward (:968-1029), memset(G),
 * backward with the MTP heads (:1036-1154), global_gradnorm and AdamW with
 * the clip folded in.  All work is issued on one stream; the host copies
 * tokens in and reads the loss out at step boundaries only.
 *
 * Scope: dense FFN or top-1 MoE layers (K = 1, no router bias), no QK-norm,
 * head_dim 32, full causal or sliding-window attention.
 */
#ifndef TL_TRAIN_H
#define TL_TRAIN_H
#include <stddef.h>
#ifdef __cplusplus
extern "C" {
#endif

/* tinylm.c's Cfg (:35-59) fields the training step uses. */
typedef struct {
    int V, D, L, H, KV, F, T;
    int n_mtp, n_exp, win, full_every;
    float rope_base;
    int qknorm;             /* QK-norm gains (tinylm.c Cfg :52): decode only, the
                               reference refuses to train such models (:2707-2713) */
} TlModel;

typedef struct TlTrain TlTrain;

/* Allocate a step for batches of B sequences (N = B*T rows).  P, M, V and
 * G start at zero.  NULL on bad shapes or allocation failure (the reason is
 * in tlg_last_error()). */
TlTrain *tl_train_new(const TlModel *m, int B);
void     tl_train_free(TlTrain *t);
size_t   tl_train_nparams(const TlTrain *t);
/* Device buffers: 0 P, 1 G, 2 AdamW M, 3 AdamW V (tl_train_nparams floats). */
float   *tl_train_buf(TlTrain *t, int which);
/* Device address of a named activation ("logits", "dlogits", "x_final",
 * "fn_norm", "a_in", "q", "k", "v", "att_ctx", "lse", "f_in", "act", ...;
 * per-layer ones at `layer`), for tests; NULL if unknown.  When H / KV is a
 * multiple of 4, "q" and "k" hold the projections before rope_apply (the
 * attention kernels rotate as they load); after a backward pass a dense
 * layer's "g" and "u" hold dg and du. */
float   *tl_train_act(TlTrain *t, const char *name, int layer);

/* Copy a host parameter vector into P and clear M and V. */
int  tl_train_upload(TlTrain *t, const float *P, void *stream);
/* Copy one batch of host tokens in: tok and tgt are N ints, tgt_mtp is
 * n_mtp x N ints (NULL when n_mtp = 0).  Tokens must lie in [0, V). */
int  tl_train_set_batch(TlTrain *t, const int *tok, const int *tgt, const int *tgt_mtp, void *stream);
/* AdamW hyper-parameters for step `step` (1-based, adamw's t): copied to the
 * device, so captured steps replay with the current values. */
int  tl_train_set_hyper(TlTrain *t, float lr, float b1, float b2, float wd, int step, void *stream);

/* A backward reads activations of the forward before it; with MoE layers it
 * also consumes their kept expert state (g, u become dg, du), so each
 * backward needs a forward of its own. */
int  tl_train_forward(TlTrain *t, void *stream);   /* loss -> device         */
int  tl_train_backward(TlTrain *t, void *stream);  /* G = d loss / d P        */
int  tl_train_optimize(TlTrain *t, void *stream);  /* gradnorm + AdamW        */
int  tl_train_step(TlTrain *t, void *stream);      /* the three above         */
/* Synchronize `stream` and read the last forward's loss / the last gradnorm. */
float tl_train_loss(TlTrain *t, void *stream);
float tl_train_gnorm(TlTrain *t, void *stream);

/* Capture tl_train_step into a HIP graph (run one eager step first so every
 * scratch buffer has its size) and replay it. */
int  tl_train_graph_build(TlTrain *t, void *stream);
int  tl_train_graph_step(TlTrain *t, void *stream);

/* Per-phase timing of one eager step: ms[0] forward, ms[1] backward,
 * ms[2] optimizer (HIP events on `stream`). */
int  tl_train_time_phases(TlTrain *t, float *ms, void *stream);
/* Tile configuration of each grouped GEMM launch of the step: per launch the
 * fastest of cands (tlg_tune_group indices) over reps timed forward + backward
 * passes (the parameters and AdamW moments are untouched).  Later steps, and
 * graphs built after it, launch with that table.  tl_train_tiles copies the
 * table (cfg[k] = configuration of launch k, -1 = automatic) and returns the
 * number of launches it covers. */
#define TL_TRAIN_MAXG 512
int  tl_train_autotune(TlTrain *t, const int *cands, int ncands, int reps, void *stream);
int  tl_train_tiles(const TlTrain *t, int *cfg, int cap);
/* The same with split targets (tlg_tune_group_split values, 0 = automatic):
 * every (cands[c], rts[s]) pair is timed and each launch keeps its fastest
 * pair; tl_train_autotune is this with rts = {0}.  tl_train_splits copies the
 * split targets as tl_train_tiles copies the configurations. */
int  tl_train_autotune_split(TlTrain *t, const int *cands, int ncands, const int *rts, int nrts, int reps,
                             void *stream);
int  tl_train_splits(const TlTrain *t, int *rt, int cap);

#ifdef __cplusplus
}
#endif
#endif
