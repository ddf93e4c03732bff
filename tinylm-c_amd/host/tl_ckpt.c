/* tl_ckpt.c -- tinylm.c model files; the format is described in tl_ckpt.h. */
#define _FILE_OFFSET_BITS 64
#define _POSIX_C_SOURCE 200809L
#include "tl_ckpt.h"

#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include <sys/types.h>

/* header ints by version (hdr_ints, tinylm.c:1692-1700) */
static const int k_hdr_ints[8] = {0, 8, 9, 10, 11, 13, 15, 16};

/* param_count's terms in unsigned 128-bit arithmetic: every field is below
 * 2^31, so the largest term, L * (n_exp + n_shared) * 3 * D * F, stays below
 * 2^127 and nothing wraps here; callers refuse a total that does not fit in
 * a size_t of bytes. */
typedef unsigned __int128 u128;
static u128 param_count_wide(const TlCkpt *c)
{
    const u128 D = (u128)c->D, F = (u128)c->F, hd = (u128)(c->D / c->H);
    const u128 KD = (u128)c->KV * hd;
    const u128 slots = c->n_exp > 0 ? (u128)c->n_exp + (u128)c->n_shared : 1;
    const u128 per = D + D * D + 2 * D * KD + D * D + (c->qknorm ? 2 * hd : 0) + D +
                     (c->n_exp > 0 ? D * (u128)c->n_exp : 0) + slots * 3 * D * F;
    return (u128)c->V * D + (u128)c->L * per + D + (u128)c->n_mtp * D * D;
}

size_t tl_ckpt_param_count(const TlCkpt *c)
{
    const u128 n = param_count_wide(c);
    return n > (u128)(SIZE_MAX / 4) ? 0 : (size_t)n;
}

/* The reference derives sizes from any header (cfg_from_hdr, cfg_derive); only
 * headers whose sizes mean nothing (non-positive dimensions, negative counts)
 * or whose parameter count does not fit in memory addresses are refused. */
static int shape_ok(const TlCkpt *c)
{
    if (c->V <= 0 || c->D <= 0 || c->L <= 0 || c->H <= 0 || c->KV <= 0 || c->F <= 0 || c->T <= 0) return 0;
    if (c->n_mtp < 0 || c->n_exp < 0 || c->n_shared < 0 || c->win < 0 || c->full_every < 0 || c->topk < 0)
        return 0;
    const u128 n = param_count_wide(c);
    return n >= 1 && n <= (u128)(SIZE_MAX / 4);
}

static void fill_fields(TlCkpt *c, const int32_t *h)
{
    c->V = h[0]; c->D = h[1]; c->L = h[2]; c->H = h[3];
    c->KV = h[4]; c->F = h[5]; c->T = h[6]; c->eot = h[7];
    if (c->version >= 2) c->tmpl = h[8];
    if (c->version >= 3) c->n_mtp = h[9];
    if (c->version >= 4) c->n_exp = h[10];
    if (c->version >= 5) { c->win = h[11]; c->full_every = h[12]; }
    if (c->version >= 6) { c->n_shared = h[13]; c->qknorm = h[14]; }
    if (c->version >= 7) c->topk = h[15];
}

int tl_ckpt_open(const char *path, TlCkpt *c)
{
    memset(c, 0, sizeof *c);
    c->tok_len = -1;
    FILE *f = path ? fopen(path, "rb") : NULL;
    if (!f) return TL_CKPT_EIO;
    int rc = TL_CKPT_OK;
    char m[4];
    int32_t h[16];
    off_t size = -1;
    if (fseeko(f, 0, SEEK_END) == 0) size = ftello(f);
    if (size < 0 || fseeko(f, 0, SEEK_SET) != 0) { rc = TL_CKPT_EIO; goto out; }
    if (fread(m, 1, 4, f) != 4) { rc = TL_CKPT_ETRUNC; goto out; }
    if (m[0] == 'T' && m[1] == 'L' && m[2] == 'Q' && m[3] >= '1' && m[3] <= '4') { rc = TL_CKPT_EQUANT; goto out; }
    if (!(m[0] == 'T' && m[1] == 'L' && m[2] == 'M' && m[3] >= '1' && m[3] <= '7')) { rc = TL_CKPT_EMAGIC; goto out; }
    c->version = m[3] - '0';
    const int nh = k_hdr_ints[c->version];
    if (fread(h, 4, (size_t)nh, f) != (size_t)nh) { rc = TL_CKPT_ETRUNC; goto out; }
    fill_fields(c, h);
    if (!shape_ok(c)) { rc = TL_CKPT_ESHAPE; goto out; }
    c->n_params = tl_ckpt_param_count(c);
    c->params_offset = 4 + 4 * (size_t)nh;
    /* the body must fit in what follows the header (compared without
     * forming 4 * n_params, which a crafted header could make wrap) */
    if ((uint64_t)size < (uint64_t)c->params_offset ||
        ((uint64_t)size - c->params_offset) / 4 < (uint64_t)c->n_params) { rc = TL_CKPT_ETRUNC; goto out; }
    const uint64_t end_params = (uint64_t)c->params_offset + 4 * (uint64_t)c->n_params;
    /* model_load_full reads the tokenizer length after the parameters from
     * TLM2 on, when the file still holds 4 bytes; a blob it announces must fit */
    if (c->version >= 2 && (uint64_t)size >= end_params + 4) {
        int32_t tl = 0;
        if (fseeko(f, (off_t)end_params, SEEK_SET) != 0 || fread(&tl, 4, 1, f) != 1) { rc = TL_CKPT_EIO; goto out; }
        c->tok_len = tl > 0 ? tl : 0;
        if (tl > 0 && (uint64_t)size < end_params + 4 + (uint64_t)tl) { rc = TL_CKPT_ETRUNC; goto out; }
    }
out:
    fclose(f);
    return rc;
}

int tl_ckpt_read(const char *path, const TlCkpt *c, float *P, size_t n)
{
    if (!c || !P || n < c->n_params || c->version < 1 || c->version > 7) return TL_CKPT_ESHAPE;
    FILE *f = path ? fopen(path, "rb") : NULL;
    if (!f) return TL_CKPT_EIO;
    int rc = TL_CKPT_OK;
    if (fseeko(f, (off_t)c->params_offset, SEEK_SET) != 0) rc = TL_CKPT_EIO;
    else if (fread(P, sizeof(float), c->n_params, f) != c->n_params) rc = TL_CKPT_ETRUNC;
    fclose(f);
    return rc;
}

int tl_ckpt_model(const TlCkpt *c, TlModel *m)
{
    memset(m, 0, sizeof *m);
    /* Shared experts are refused by the reference itself (check_supported,
     * :1946-1953); routing to more than one expert is not the top-1 layer
     * built here (moe_route, :814-827).  QK-norm models (TLM6/7) decode; the
     * training step refuses them, as the reference does (:2707-2713). */
    if (c->n_shared > 0 || (c->n_exp > 0 && c->topk > 1)) return TL_CKPT_EUNSUP;
    m->V = c->V; m->D = c->D; m->L = c->L; m->H = c->H;
    m->KV = c->KV; m->F = c->F; m->T = c->T;
    m->n_mtp = c->n_mtp; m->n_exp = c->n_exp;
    m->win = c->win; m->full_every = c->full_every;
    m->rope_base = 10000.0f;
    m->qknorm = c->qknorm;
    return TL_CKPT_OK;
}

const char *tl_ckpt_error(int code)
{
    switch (code) {
    case TL_CKPT_OK: return "ok";
    case TL_CKPT_EIO: return "cannot open or read the file";
    case TL_CKPT_EMAGIC: return "not a tinylm model file (magic TLM1-TLM7)";
    case TL_CKPT_EQUANT: return "quantized model file (TLQ1-TLQ4): not read by the fp32 path";
    case TL_CKPT_ESHAPE: return "header fields describe no model";
    case TL_CKPT_ETRUNC: return "file shorter than its header announces";
    case TL_CKPT_EUNSUP: return "model uses shared experts or top-k > 1 routing, which this build does not run";
    default: return "unknown error";
    }
}
