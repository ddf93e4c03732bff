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

size_t tl_ckpt_param_count(const TlCkpt *c)
{
    const size_t D = (size_t)c->D, F = (size_t)c->F, hd = (size_t)(c->D / c->H);
    const size_t KD = (size_t)c->KV * hd;
    const size_t slots = c->n_exp > 0 ? (size_t)c->n_exp + (size_t)c->n_shared : 1;
    const size_t per = D + D * D + 2 * D * KD + D * D + (c->qknorm ? 2 * hd : 0) + D +
                       (c->n_exp > 0 ? D * (size_t)c->n_exp : 0) + slots * 3 * D * F;
    return (size_t)c->V * D + (size_t)c->L * per + D + (size_t)c->n_mtp * D * D;
}

/* The reference derives sizes from any header (cfg_from_hdr, cfg_derive); only
 * headers whose sizes mean nothing (non-positive dimensions, negative counts,
 * sizes that would overflow) are refused here. */
static int shape_ok(const TlCkpt *c)
{
    if (c->V <= 0 || c->D <= 0 || c->L <= 0 || c->H <= 0 || c->KV <= 0 || c->F <= 0 || c->T <= 0) return 0;
    if (c->n_mtp < 0 || c->n_exp < 0 || c->n_shared < 0 || c->win < 0 || c->full_every < 0 || c->topk < 0)
        return 0;
    /* keep every product in param_count far from size_t overflow */
    const int64_t big = (int64_t)1 << 24;
    if (c->V > big || c->D > big || c->F > big || c->L > 65536 || c->n_exp > 65536 || c->n_shared > 65536 ||
        c->n_mtp > 65536)
        return 0;
    return 1;
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
    const uint64_t end_params = (uint64_t)c->params_offset + 4 * (uint64_t)c->n_params;
    if ((uint64_t)size < end_params) { rc = TL_CKPT_ETRUNC; goto out; }
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

void tl_ckpt_model(const TlCkpt *c, TlModel *m)
{
    memset(m, 0, sizeof *m);
    m->V = c->V; m->D = c->D; m->L = c->L; m->H = c->H;
    m->KV = c->KV; m->F = c->F; m->T = c->T;
    m->n_mtp = c->n_mtp; m->n_exp = c->n_exp;
    m->win = c->win; m->full_every = c->full_every;
    m->rope_base = 10000.0f;
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
    default: return "unknown error";
    }
}
