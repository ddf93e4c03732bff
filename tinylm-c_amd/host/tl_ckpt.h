/* tl_ckpt.h -- reading tinylm.c model files (libtlhost.so, plain C).
 *
 * The reference's fp32 checkpoints (written by model_save_bundle,
 * tinylm.c:1895-1913; read by model_load / model_load_full, :1915-1983):
 *   4-byte magic "TLM1" .. "TLM7"
 *   int32 header fields, 8 / 9 / 10 / 11 / 13 / 15 / 16 of them by version
 *     (hdr_ints :1691-1700; their meaning, cfg_from_hdr :1705-1718):
 *     V D L H KV F T eot | tmpl (TLM2+) | n_mtp (TLM3+) | n_exp (TLM4+) |
 *     win full_every (TLM5+) | n_shared qknorm (TLM6+) | topk (TLM7)
 *   param_count(cfg) float32 parameters in map_weights' order (:345-393)
 *   from TLM2 on: an int32 tokenizer length and the tokenizer blob.
 * The parameters are the flat P that the training step, the GEMM plans and
 * the decoder of this library take (tl_train.h, tl_decode.h).  Quantized
 * files (TLQ1-TLQ4) are refused: their dequantisation belongs to the int8
 * decode path, which this build does not cover.
 */
#ifndef TL_CKPT_H
#define TL_CKPT_H
#include <stddef.h>
#include "tl_train.h"
#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int version;                      /* 1 .. 7 */
    int V, D, L, H, KV, F, T, eot;    /* every version */
    int tmpl, n_mtp, n_exp;           /* TLM2+, TLM3+, TLM4+ (0 before) */
    int win, full_every;              /* TLM5+ */
    int n_shared, qknorm;             /* TLM6+ */
    int topk;                         /* TLM7 */
    size_t n_params;                  /* param_count of the header's model */
    size_t params_offset;             /* byte offset of the parameters in the file */
    long long tok_len;                /* tokenizer blob bytes; -1 when none is recorded */
} TlCkpt;

#define TL_CKPT_OK      0
#define TL_CKPT_EIO    -1             /* cannot open or read the file */
#define TL_CKPT_EMAGIC -2             /* not a TLM1-TLM7 file */
#define TL_CKPT_EQUANT -3             /* a quantized TLQ1-TLQ4 file */
#define TL_CKPT_ESHAPE -4             /* header fields that describe no model */
#define TL_CKPT_ETRUNC -5             /* the file ends before what its header announces */
#define TL_CKPT_EUNSUP -6             /* a model the step / decoder here cannot run */

/* Parse the header of `path` into *c and check that the file holds the
 * parameters (and the tokenizer blob it announces).  TL_CKPT_OK or an error
 * code; *c is zeroed first. */
int tl_ckpt_open(const char *path, TlCkpt *c);

/* param_count (tinylm.c:345-358) of the model c describes: embedding, per
 * layer an1, Wq, Wk, Wv, Wo, the QK-norm gains when qknorm, an2, the router
 * when n_exp > 0, the FFN of every expert slot (n_exp + n_shared routed and
 * shared experts, or 1 dense FFN), then the final norm and the n_mtp heads.
 * 0 when the count times 4 bytes does not fit in a size_t. */
size_t tl_ckpt_param_count(const TlCkpt *c);

/* Read the c->n_params parameters of `path` (opened by tl_ckpt_open) into P,
 * which holds n >= c->n_params floats.  TL_CKPT_OK or an error code. */
int tl_ckpt_read(const char *path, const TlCkpt *c, float *P, size_t n);

/* The model fields the training step and the decoder take (rope_base 10000,
 * as cfg_from_hdr sets it; qknorm as the header says: the decoder runs it,
 * the training step refuses it as the reference does).  TL_CKPT_OK, or
 * TL_CKPT_EUNSUP (and *m zeroed) for a model they would misread: shared
 * experts (n_shared > 0, which the reference refuses too) or MoE routing to
 * topk > 1 experts. */
int tl_ckpt_model(const TlCkpt *c, TlModel *m);

/* A short text for an error code. */
const char *tl_ckpt_error(int code);

#ifdef __cplusplus
}
#endif
#endif
