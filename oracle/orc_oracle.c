/*
 * orc_oracle.c — CPU restatement of ORACLE's speculative-decoding hot path.
 * TEST INFRASTRUCTURE ONLY (see orc_oracle.h). Reference file:line cited per
 * function; paths are relative to the reference tree.
 *
 * Build: oracle/Makefile compiles this with -ffp-contract=off so that every
 * fused multiply-add below is an explicit fmaf(), matching what the reference
 * build does where g++ contracts or where AVX2 intrinsics use FMA.
 */
#define _GNU_SOURCE
#include "orc_oracle.h"

#include <fcntl.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

/* ── fp16 (gguf_parser.cpp:1002-1022) ─────────────────────────────────────── */
float orco_fp16(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) & 1u, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu, f;
    if (e == 0) {
        if (m == 0) f = sign << 31;
        else {
            uint32_t k = 0;
            while (!(m & 0x400u)) { m <<= 1; k++; }
            f = (sign << 31) | ((127u - 15u - k + 1u) << 23) | ((m & 0x3FFu) << 13);
        }
    } else if (e == 31) f = (sign << 31) | (0xFFu << 23) | (m << 13);
    else f = (sign << 31) | ((e + 127u - 15u) << 23) | (m << 13);
    float r;
    memcpy(&r, &f, 4);
    return r;
}
static inline float rd_h(const uint8_t* p) { uint16_t h; memcpy(&h, p, 2); return orco_fp16(h); }

uint64_t orco_row_bytes(int type, int64_t n) {
    switch (type) {
        case ORCO_F32: return (uint64_t)n * 4;
        case ORCO_F16: case ORCO_BF16: return (uint64_t)n * 2;
        case ORCO_Q4_0: return (uint64_t)(n / 32) * 18;
        case ORCO_Q8_0: return (uint64_t)(n / 32) * 34;
        case ORCO_Q4_K: return (uint64_t)(n / 256) * 144;
        case ORCO_Q6_K: return (uint64_t)(n / 256) * 210;
        default: return 0;
    }
}

/* ── dequant codecs (gguf_parser.cpp:1029-1154) ─────────────────────────────
 * Rounding as compiled by the reference build: Q4_0/Q8_0 one product; Q4_K
 * d1*q - m1f contracted into one FMA (verified against the reference's
 * test_dq_q4_k hook); Q6_K (d*sc)*q with two roundings. */
static void scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) { /* :1085-1093 */
    if (j < 4) { *d = q[j] & 63; *m = q[j + 4] & 63; }
    else {
        *d = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

int orco_dequant(int type, const uint8_t* s, int64_t n, float* out) {
    switch (type) {
    case ORCO_F32: memcpy(out, s, (size_t)n * 4); return 0;
    case ORCO_F16: for (int64_t i = 0; i < n; i++) out[i] = rd_h(s + 2 * i); return 0;
    case ORCO_BF16:
        for (int64_t i = 0; i < n; i++) { uint16_t b; memcpy(&b, s + 2 * i, 2); uint32_t f = (uint32_t)b << 16; memcpy(out + i, &f, 4); }
        return 0;
    case ORCO_Q4_0: /* :1058-1070 */
        for (int64_t b = 0; b < n / 32; b++) {
            const uint8_t* blk = s + b * 18;
            float d = rd_h(blk);
            for (int l = 0; l < 16; l++) {
                out[b * 32 + l] = d * (float)((int)(blk[2 + l] & 0xF) - 8);
                out[b * 32 + l + 16] = d * (float)((int)(blk[2 + l] >> 4) - 8);
            }
        }
        return 0;
    case ORCO_Q8_0: /* :1073-1082 */
        for (int64_t b = 0; b < n / 32; b++) {
            const uint8_t* blk = s + b * 34;
            float d = rd_h(blk);
            for (int l = 0; l < 32; l++) out[b * 32 + l] = d * (float)(int8_t)blk[2 + l];
        }
        return 0;
    case ORCO_Q4_K: /* :1096-1121 */
        for (int64_t b = 0; b < n / 256; b++) {
            const uint8_t* blk = s + b * 144;
            float d = rd_h(blk), dmin = rd_h(blk + 2);
            const uint8_t* sc = blk + 4;
            const uint8_t* qs = blk + 16;
            float* dst = out + b * 256;
            for (int j = 0, is = 0; j < 256; j += 64, is += 2, qs += 32) {
                uint8_t s0, m0, s1, m1;
                scale_min_k4(is, sc, &s0, &m0);
                scale_min_k4(is + 1, sc, &s1, &m1);
                float d1 = d * s0, m1f = dmin * m0, d2 = d * s1, m2f = dmin * m1;
                for (int l = 0; l < 32; l++) {
                    dst[j + l] = fmaf(d1, (float)(qs[l] & 0xF), -m1f);
                    dst[j + 32 + l] = fmaf(d2, (float)(qs[l] >> 4), -m2f);
                }
            }
        }
        return 0;
    case ORCO_Q6_K: /* :1124-1154 */
        for (int64_t b = 0; b < n / 256; b++) {
            const uint8_t* blk = s + b * 210;
            const uint8_t* ql = blk;
            const uint8_t* qh = blk + 128;
            const int8_t* sc = (const int8_t*)(blk + 192);
            float d = rd_h(blk + 208);
            float* dst = out + b * 256;
            for (int j = 0; j < 256; j += 128, ql += 64, qh += 32, sc += 8) {
                for (int l = 0; l < 32; l++) {
                    int is = l / 16;
                    int q1 = ((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                    int q2 = ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                    int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                    int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                    dst[j + l] = (d * (float)sc[is + 0]) * (float)q1;
                    dst[j + l + 32] = (d * (float)sc[is + 2]) * (float)q2;
                    dst[j + l + 64] = (d * (float)sc[is + 4]) * (float)q3;
                    dst[j + l + 96] = (d * (float)sc[is + 6]) * (float)q4;
                }
            }
        }
        return 0;
    default: return -1;
    }
}

/* ── quantized row dots, decode path (gguf_parser.cpp:496-866) ───────────── */
float orco_dot(int type, const uint8_t* row, int n, const float* x) {
    float acc = 0.f;
    switch (type) {
    case ORCO_Q8_0: /* :496-551  acc = fma(d*q, x, acc) */
        for (int b = 0; b < n / 32; b++) {
            const uint8_t* blk = row + b * 34;
            float d = rd_h(blk);
            for (int l = 0; l < 32; l++) acc = fmaf(d * (float)(int8_t)blk[2 + l], x[b * 32 + l], acc);
        }
        return acc;
    case ORCO_Q4_0: /* :556-631  per block acc = fma(d, sum_lo + sum_hi, acc) */
        for (int b = 0; b < n / 32; b++) {
            const uint8_t* blk = row + b * 18;
            float d = rd_h(blk), sl = 0.f, sh = 0.f;
            for (int l = 0; l < 16; l++) {
                sl = fmaf((float)((int)(blk[2 + l] & 0xF) - 8), x[b * 32 + l], sl);
                sh = fmaf((float)((int)(blk[2 + l] >> 4) - 8), x[b * 32 + l + 16], sh);
            }
            acc = fmaf(d, sl + sh, acc);
        }
        return acc;
    case ORCO_Q4_K: /* :635-719  acc += d1*s1 - m1f*sx1 + d2*s2 - m2f*sx2 per 64 */
        for (int b = 0; b < n / 256; b++) {
            const uint8_t* blk = row + b * 144;
            float d = rd_h(blk), dmin = rd_h(blk + 2);
            const uint8_t* qs = blk + 16;
            const float* xb = x + b * 256;
            for (int j = 0, is = 0; j < 256; j += 64, is += 2, qs += 32) {
                uint8_t s0, m0, s1, m1;
                scale_min_k4(is, blk + 4, &s0, &m0);
                scale_min_k4(is + 1, blk + 4, &s1, &m1);
                float d1 = d * s0, m1f = dmin * m0, d2 = d * s1, m2f = dmin * m1;
                float s1v = 0.f, s2v = 0.f, sx1 = 0.f, sx2 = 0.f;
                for (int l = 0; l < 32; l++) {
                    s1v = fmaf((float)(qs[l] & 0xF), xb[j + l], s1v);
                    s2v = fmaf((float)(qs[l] >> 4), xb[j + 32 + l], s2v);
                    sx1 += xb[j + l];
                    sx2 += xb[j + 32 + l];
                }
                acc += d1 * s1v - m1f * sx1 + d2 * s2v - m2f * sx2;
            }
        }
        return acc;
    case ORCO_Q6_K: /* :721-866  acc = fma((d*sc)*q, x, acc) */
        for (int b = 0; b < n / 256; b++) {
            const uint8_t* blk = row + b * 210;
            const uint8_t* ql = blk;
            const uint8_t* qh = blk + 128;
            const int8_t* sc = (const int8_t*)(blk + 192);
            float d = rd_h(blk + 208);
            const float* xb = x + b * 256;
            for (int j = 0; j < 256; j += 128, ql += 64, qh += 32, sc += 8) {
                for (int l = 0; l < 32; l++) {
                    int is = l / 16;
                    int q1 = ((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                    int q2 = ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                    int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                    int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                    acc = fmaf((d * (float)sc[is + 0]) * (float)q1, xb[j + l], acc);
                    acc = fmaf((d * (float)sc[is + 2]) * (float)q2, xb[j + l + 32], acc);
                    acc = fmaf((d * (float)sc[is + 4]) * (float)q3, xb[j + l + 64], acc);
                    acc = fmaf((d * (float)sc[is + 6]) * (float)q4, xb[j + l + 96], acc);
                }
            }
        }
        return acc;
    default: {
        /* F32/F16/BF16: the reference falls back to dequant + ops::matmul (model.cpp:370-381) */
        float* w = (float*)malloc(sizeof(float) * (size_t)n);
        orco_dequant(type, row, n, w);
        for (int i = 0; i < n; i++) acc = fmaf(w[i], x[i], acc);
        free(w);
        return acc;
    }
    }
}

int orco_gemv(int type, const uint8_t* w, int n_out, int n_in, const float* x, float* y) { /* :873-911 */
    uint64_t rb = orco_row_bytes(type, n_in);
    if (!rb) return -1;
    for (int j = 0; j < n_out; j++) y[j] = orco_dot(type, w + (uint64_t)j * rb, n_in, x);
    return 0;
}

/* ops::dot (ops.cpp:102-143) */
static float dotf(const float* a, const float* b, int n) {
    float s = 0.f;
    for (int i = 0; i < n; i++) s = fmaf(a[i], b[i], s);
    return s;
}

int orco_gemm(int type, const uint8_t* w, int n_tok, int n_out, int n_in, const float* x, float* y) { /* :919-997 */
    uint64_t rb = orco_row_bytes(type, n_in);
    if (!rb) return -1;
    float* row = (float*)malloc(sizeof(float) * (size_t)n_in);
    for (int j = 0; j < n_out; j++) {
        orco_dequant(type, w + (uint64_t)j * rb, n_in, row);
        for (int t = 0; t < n_tok; t++) y[(size_t)t * n_out + j] = dotf(x + (size_t)t * n_in, row, n_in);
    }
    free(row);
    return 0;
}

/* ── elementwise ops (ops.cpp) ───────────────────────────────────────────── */
void orco_rmsnorm(float* out, const float* x, const float* w, int n, float eps) { /* :149-195 */
    float ss = 0.f;
    for (int i = 0; i < n; i++) ss = fmaf(x[i], x[i], ss);
    ss = 1.f / sqrtf(ss / (float)n + eps);
    for (int i = 0; i < n; i++) out[i] = (x[i] * ss) * w[i];
}

void orco_rope(float* q, float* k, int nh, int nkv, int hd, int pos, float base) { /* :440-485 */
    int half = hd / 2;
    float cs[512], sn[512];
    for (int i = 0; i < half; i++) {
        float th = (float)pos / powf(base, (float)(2 * i) / (float)hd);
        cs[i] = cosf(th);
        sn[i] = sinf(th);
    }
    for (int h = 0; h < nh + nkv; h++) {
        float* v = h < nh ? q + h * hd : k + (h - nh) * hd;
        for (int i = 0; i < half; i++) {
            float a = v[i], b = v[i + half];
            v[i] = a * cs[i] - b * sn[i];
            v[i + half] = a * sn[i] + b * cs[i];
        }
    }
}

void orco_softmax(float* x, int n) { /* :386-435 */
    if (n <= 0) return;
    float mx = x[0], sum = 0.f;
    for (int i = 1; i < n; i++) if (x[i] > mx) mx = x[i];
    for (int i = 0; i < n; i++) { x[i] = expf(x[i] - mx); sum += x[i]; }
    float inv = 1.f / sum;
    for (int i = 0; i < n; i++) x[i] *= inv;
}

void orco_silu(float* x, int n) { /* :308-334 */
    for (int i = 0; i < n; i++) x[i] = x[i] / (1.f + expf(-x[i]));
}

int orco_argmax(const float* x, int n) { /* :490-497 */
    if (n <= 0) return 0;
    int best = 0;
    float v = x[0];
    for (int i = 1; i < n; i++) if (x[i] > v) { v = x[i]; best = i; }
    return best;
}

void orco_attention(const float* q, const float* kc, const float* vc, int nh, int nkv, int hd, int pos,
                    float* out) { /* model.cpp:410-435 */
    const int nkvt = nkv * hd, gqa = nh / nkv;
    const float scale = 1.f / sqrtf((float)hd);
    float* att = (float*)malloc(sizeof(float) * (size_t)(pos + 1));
    for (int h = 0; h < nh; h++) {
        const int g = h / gqa;
        const float* qh = q + h * hd;
        float* oh = out + h * hd;
        for (int t = 0; t <= pos; t++) att[t] = dotf(qh, kc + (size_t)t * nkvt + g * hd, hd) * scale;
        orco_softmax(att, pos + 1);
        for (int i = 0; i < hd; i++) oh[i] = 0.f;
        for (int t = 0; t <= pos; t++) {
            const float* vh = vc + (size_t)t * nkvt + g * hd;
            for (int i = 0; i < hd; i++) oh[i] = fmaf(att[t], vh[i], oh[i]);
        }
    }
    free(att);
}

/* ── minimal GGUF reader (gguf_parser.cpp:164-324) ───────────────────────── */
typedef struct { char name[128]; int type; int ndim; uint64_t shape[8]; uint64_t off; } otensor;
typedef struct { int type; const uint8_t* p; int n_in, n_out; } omat;

struct orco_model {
    uint8_t* map; size_t size; const uint8_t* data;
    otensor* t; int nt;
    char arch[64];
    int V, L, H, KVH, D, FF, HD, CTX, NQ, NKV, bias, tied, qkn;
    float rope, eps;  /* eps: attention.layer_norm_rms_epsilon, used by the QK-norm only */
    omat embd, head, *wq, *wk, *wv, *wo, *wg, *wu, *wd;
    const float **attn_norm, **ffn_norm, *out_norm, **bq, **bk, **bv, **qn, **kn;
    float *kc, *vc, *x, *xb, *xb2, *hb, *hb2, *q, *k, *v, *att;
};

typedef struct { const uint8_t* p; const uint8_t* end; int ok; } rdr;
static uint64_t rdu(rdr* r, int n) {
    uint64_t v = 0;
    if (r->p + n > r->end) { r->ok = 0; return 0; }
    memcpy(&v, r->p, (size_t)n);
    r->p += n;
    return v;
}
static void rds(rdr* r, char* dst, size_t cap) {
    uint64_t n = rdu(r, 8);
    if (!r->ok || n > (uint64_t)(r->end - r->p)) { r->ok = 0; return; }
    if (dst) { size_t c = n < cap - 1 ? (size_t)n : cap - 1; memcpy(dst, r->p, c); dst[c] = 0; }
    r->p += n;
}
static const int kv_size[] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};

typedef struct { char key[160]; int kind; uint64_t u; float f; char s[64]; } okv;

static void skip_value(rdr* r, int kind) {
    if (kind == 8) { rds(r, NULL, 0); return; }
    if (kind == 9) {
        int at = (int)rdu(r, 4);
        uint64_t n = rdu(r, 8);
        for (uint64_t i = 0; i < n && r->ok; i++) skip_value(r, at);
        return;
    }
    if (kind < 0 || kind > 12) { r->ok = 0; return; }
    r->p += kv_size[kind];
    if (r->p > r->end) r->ok = 0;
}

static const otensor* find_t(const orco_model* m, const char* name) {
    for (int i = 0; i < m->nt; i++) if (!strcmp(m->t[i].name, name)) return &m->t[i];
    return NULL;
}

static int get_mat(orco_model* m, const char* name, omat* o) {
    const otensor* t = find_t(m, name);
    if (!t) return -1;
    o->type = t->type;
    o->p = m->data + t->off;
    o->n_in = (int)t->shape[0];
    o->n_out = t->ndim > 1 ? (int)t->shape[1] : 1;
    return 0;
}
static const float* get_vec(orco_model* m, const char* name) {
    const otensor* t = find_t(m, name);
    return t ? (const float*)(m->data + t->off) : NULL;
}

orco_model* orco_model_load(const char* path, int ctx_len) {
    int fd = open(path, O_RDONLY);
    if (fd < 0) return NULL;
    struct stat st;
    if (fstat(fd, &st) < 0) { close(fd); return NULL; }
    uint8_t* map = (uint8_t*)mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) return NULL;
    orco_model* m = (orco_model*)calloc(1, sizeof(orco_model));
    m->map = map;
    m->size = (size_t)st.st_size;
    rdr r = {map, map + st.st_size, 1};
    if (st.st_size < 24 || memcmp(map, "GGUF", 4)) goto fail;
    r.p += 4;
    rdu(&r, 4);
    uint64_t nt = rdu(&r, 8), nkv = rdu(&r, 8);
    okv* kvs = (okv*)calloc((size_t)nkv + 1, sizeof(okv));
    for (uint64_t i = 0; i < nkv && r.ok; i++) {
        rds(&r, kvs[i].key, sizeof kvs[i].key);
        int kind = (int)rdu(&r, 4);
        kvs[i].kind = kind;
        if (kind == 8) rds(&r, kvs[i].s, sizeof kvs[i].s);
        else if (kind == 4 || kind == 5) kvs[i].u = rdu(&r, 4);
        else if (kind == 10) kvs[i].u = rdu(&r, 8);
        else if (kind == 6) { uint32_t b = (uint32_t)rdu(&r, 4); memcpy(&kvs[i].f, &b, 4); }
        else if (kind == 12) { uint64_t b = rdu(&r, 8); double dv; memcpy(&dv, &b, 8); kvs[i].f = (float)dv; }
        else skip_value(&r, kind);
    }
    m->t = (otensor*)calloc((size_t)nt + 1, sizeof(otensor));
    m->nt = (int)nt;
    for (uint64_t i = 0; i < nt && r.ok; i++) {
        rds(&r, m->t[i].name, sizeof m->t[i].name);
        m->t[i].ndim = (int)rdu(&r, 4);
        if (m->t[i].ndim > 8) { r.ok = 0; break; }
        for (int d = 0; d < m->t[i].ndim; d++) m->t[i].shape[d] = rdu(&r, 8);
        m->t[i].type = (int)rdu(&r, 4);
        m->t[i].off = rdu(&r, 8);
    }
    if (!r.ok) { free(kvs); goto fail; }
    m->data = map + (((uint64_t)(r.p - map) + 31) & ~(uint64_t)31);
    /* config derivation, model.cpp:48-80 */
    strcpy(m->arch, "llama");
    for (uint64_t i = 0; i < nkv; i++) if (!strcmp(kvs[i].key, "general.architecture") && kvs[i].kind == 8) strcpy(m->arch, kvs[i].s);
#define META_U(suffix, def, dst) do { char kk[200]; snprintf(kk, sizeof kk, "%s.%s", m->arch, suffix); dst = def; \
        for (uint64_t i = 0; i < nkv; i++) if (!strcmp(kvs[i].key, kk) && (kvs[i].kind == 4 || kvs[i].kind == 5 || kvs[i].kind == 10)) dst = (int)kvs[i].u; } while (0)
    META_U("block_count", 32, m->L);
    META_U("attention.head_count", 32, m->H);
    META_U("attention.head_count_kv", m->H, m->KVH);
    META_U("embedding_length", 4096, m->D);
    META_U("feed_forward_length", 11008, m->FF);
    META_U("attention.key_length", m->D / m->H, m->HD);
    m->rope = 500000.f;
    {
        char kk[200];
        snprintf(kk, sizeof kk, "%s.rope.freq_base", m->arch);
        for (uint64_t i = 0; i < nkv; i++) if (!strcmp(kvs[i].key, kk) && (kvs[i].kind == 6 || kvs[i].kind == 12)) m->rope = kvs[i].f;
    }
    m->eps = 1e-5f;
    {
        char kk[200];
        snprintf(kk, sizeof kk, "%s.attention.layer_norm_rms_epsilon", m->arch);
        for (uint64_t i = 0; i < nkv; i++) if (!strcmp(kvs[i].key, kk) && (kvs[i].kind == 6 || kvs[i].kind == 12)) m->eps = kvs[i].f;
    }
#undef META_U
    free(kvs);
    m->CTX = ctx_len;
    m->NQ = m->H * m->HD;
    m->NKV = m->KVH * m->HD;
    const otensor* to = find_t(m, "output.weight");
    const otensor* te = find_t(m, "token_embd.weight");
    if (!te) goto fail;
    {
        const otensor* tv = to ? to : te;
        m->V = (int)(tv->shape[0] > tv->shape[1] ? tv->shape[0] : tv->shape[1]);
    }
    m->tied = to == NULL;
    get_mat(m, "token_embd.weight", &m->embd);
    get_mat(m, to ? "output.weight" : "token_embd.weight", &m->head);
    m->out_norm = get_vec(m, "output_norm.weight");
    m->bias = find_t(m, "blk.0.attn_q.bias") != NULL;
    m->qkn = find_t(m, "blk.0.attn_q_norm.weight") != NULL; /* Qwen3 QK-norm, model.cpp:63 */
#define ALLOCL(p, T) p = (T*)calloc((size_t)m->L, sizeof(T))
    ALLOCL(m->wq, omat); ALLOCL(m->wk, omat); ALLOCL(m->wv, omat); ALLOCL(m->wo, omat);
    ALLOCL(m->wg, omat); ALLOCL(m->wu, omat); ALLOCL(m->wd, omat);
    ALLOCL(m->attn_norm, const float*); ALLOCL(m->ffn_norm, const float*);
    ALLOCL(m->bq, const float*); ALLOCL(m->bk, const float*); ALLOCL(m->bv, const float*);
    ALLOCL(m->qn, const float*); ALLOCL(m->kn, const float*);
#undef ALLOCL
    for (int l = 0; l < m->L; l++) {
        char nm[128];
#define MAT(field, suffix) snprintf(nm, sizeof nm, "blk.%d.%s", l, suffix); if (get_mat(m, nm, &m->field[l])) goto fail
        MAT(wq, "attn_q.weight"); MAT(wk, "attn_k.weight"); MAT(wv, "attn_v.weight"); MAT(wo, "attn_output.weight");
        MAT(wg, "ffn_gate.weight"); MAT(wu, "ffn_up.weight"); MAT(wd, "ffn_down.weight");
#undef MAT
#define VEC(field, suffix) snprintf(nm, sizeof nm, "blk.%d.%s", l, suffix); m->field[l] = get_vec(m, nm)
        VEC(attn_norm, "attn_norm.weight"); VEC(ffn_norm, "ffn_norm.weight");
        VEC(bq, "attn_q.bias"); VEC(bk, "attn_k.bias"); VEC(bv, "attn_v.bias");
        VEC(qn, "attn_q_norm.weight"); VEC(kn, "attn_k_norm.weight");
        if (m->qkn && (!m->qn[l] || !m->kn[l])) goto fail;
#undef VEC
    }
    {
        size_t kvn = (size_t)m->L * m->CTX * m->NKV;
        m->kc = (float*)calloc(kvn, sizeof(float));
        m->vc = (float*)calloc(kvn, sizeof(float));
        int big = m->D > m->NQ ? m->D : m->NQ;
        m->x = (float*)calloc((size_t)big, sizeof(float));
        m->xb = (float*)calloc((size_t)big, sizeof(float));
        m->xb2 = (float*)calloc((size_t)big, sizeof(float));
        m->hb = (float*)calloc((size_t)m->FF, sizeof(float));
        m->hb2 = (float*)calloc((size_t)m->FF, sizeof(float));
        m->q = (float*)calloc((size_t)m->NQ, sizeof(float));
        m->k = (float*)calloc((size_t)m->NKV, sizeof(float));
        m->v = (float*)calloc((size_t)m->NKV, sizeof(float));
    }
    return m;
fail:
    orco_model_free(m);
    return NULL;
}

void orco_model_free(orco_model* m) {
    if (!m) return;
    if (m->map) munmap(m->map, m->size);
    free(m->t); free(m->wq); free(m->wk); free(m->wv); free(m->wo); free(m->wg); free(m->wu); free(m->wd);
    free(m->attn_norm); free(m->ffn_norm); free(m->bq); free(m->bk); free(m->bv); free(m->qn); free(m->kn);
    free(m->kc); free(m->vc); free(m->x); free(m->xb); free(m->xb2); free(m->hb); free(m->hb2);
    free(m->q); free(m->k); free(m->v);
    free(m);
}

void orco_model_cfg(const orco_model* m, int32_t* c, float* rope) {
    c[0] = m->V; c[1] = m->L; c[2] = m->H; c[3] = m->KVH; c[4] = m->D; c[5] = m->FF; c[6] = m->HD;
    c[7] = m->CTX; c[8] = m->bias; c[9] = m->tied;
    if (rope) *rope = m->rope;
}

void orco_model_reset(orco_model* m) {
    size_t kvn = (size_t)m->L * m->CTX * m->NKV;
    memset(m->kc, 0, kvn * sizeof(float));
    memset(m->vc, 0, kvn * sizeof(float));
}

const float* orco_model_hidden(const orco_model* m) { return m->x; }

static void embed_row(orco_model* m, int32_t tok, float* out) { /* model.cpp:352-358 */
    if (tok < 0 || tok >= m->V) tok = 0;
    uint64_t rb = orco_row_bytes(m->embd.type, m->D);
    orco_dequant(m->embd.type, m->embd.p + (uint64_t)tok * rb, m->D, out);
}

static void gemv_m(const omat* w, const float* x, float* y) { orco_gemv(w->type, w->p, w->n_out, w->n_in, x, y); }
static void addv(float* a, const float* b, int n) { for (int i = 0; i < n; i++) a[i] += b[i]; }

/* QK-norm (Qwen3): ops::rmsnorm over each q head and each k head of one
 * token, with the model's epsilon, after the bias and before RoPE
 * (model.cpp:390-399, 584-593) */
static void qk_norm(const orco_model* m, int l, float* q, float* k) {
    if (!m->qkn) return;
    for (int h = 0; h < m->H; h++) orco_rmsnorm(q + h * m->HD, q + h * m->HD, m->qn[l], m->HD, m->eps);
    for (int h = 0; h < m->KVH; h++) orco_rmsnorm(k + h * m->HD, k + h * m->HD, m->kn[l], m->HD, m->eps);
}

int orco_model_forward(orco_model* m, int32_t token, int pos, float* logits) { /* model.cpp:340-495 */
    if (pos < 0 || pos >= m->CTX) return -1;
    const int D = m->D, NQ = m->NQ, NKV = m->NKV, FF = m->FF;
    embed_row(m, token, m->x);
    for (int l = 0; l < m->L; l++) {
        orco_rmsnorm(m->xb, m->x, m->attn_norm[l], D, 1e-5f);
        gemv_m(&m->wq[l], m->xb, m->q);
        gemv_m(&m->wk[l], m->xb, m->k);
        gemv_m(&m->wv[l], m->xb, m->v);
        if (m->bias) { addv(m->q, m->bq[l], NQ); addv(m->k, m->bk[l], NKV); addv(m->v, m->bv[l], NKV); }
        qk_norm(m, l, m->q, m->k);
        orco_rope(m->q, m->k, m->H, m->KVH, m->HD, pos, m->rope);
        float* kcl = m->kc + (size_t)l * m->CTX * NKV;
        float* vcl = m->vc + (size_t)l * m->CTX * NKV;
        memcpy(kcl + (size_t)pos * NKV, m->k, sizeof(float) * NKV);
        memcpy(vcl + (size_t)pos * NKV, m->v, sizeof(float) * NKV);
        orco_attention(m->q, kcl, vcl, m->H, m->KVH, m->HD, pos, m->xb);
        gemv_m(&m->wo[l], m->xb, m->xb2);
        addv(m->x, m->xb2, D);
        orco_rmsnorm(m->xb, m->x, m->ffn_norm[l], D, 1e-5f);
        gemv_m(&m->wg[l], m->xb, m->hb);
        gemv_m(&m->wu[l], m->xb, m->hb2);
        orco_silu(m->hb, FF);
        for (int i = 0; i < FF; i++) m->hb[i] = m->hb[i] * m->hb2[i];
        gemv_m(&m->wd[l], m->hb, m->xb);
        addv(m->x, m->xb, D);
    }
    if (!logits) return 0;
    orco_rmsnorm(m->x, m->x, m->out_norm, D, 1e-5f);
    gemv_m(&m->head, m->x, logits);
    return 0;
}

int orco_model_forward_batch(orco_model* m, const int32_t* toks, int n, int sp, float* logits) { /* model.cpp:510-674 */
    if (n <= 0) return 0;
    if (sp < 0 || sp + n > m->CTX) return -1;
    const int D = m->D, NQ = m->NQ, NKV = m->NKV, FF = m->FF;
    float* X = (float*)calloc((size_t)n * D, 4);
    float* Xn = (float*)calloc((size_t)n * D, 4);
    float* Q = (float*)calloc((size_t)n * NQ, 4);
    float* K = (float*)calloc((size_t)n * NKV, 4);
    float* Vv = (float*)calloc((size_t)n * NKV, 4);
    float* AO = (float*)calloc((size_t)n * NQ, 4);
    float* XO = (float*)calloc((size_t)n * D, 4);
    float* G = (float*)calloc((size_t)n * FF, 4);
    float* U = (float*)calloc((size_t)n * FF, 4);
#define GEMM(w, in, out) orco_gemm((w)->type, (w)->p, n, (w)->n_out, (w)->n_in, in, out)
    for (int t = 0; t < n; t++) embed_row(m, toks[t], X + (size_t)t * D);
    for (int l = 0; l < m->L; l++) {
        for (int t = 0; t < n; t++) orco_rmsnorm(Xn + (size_t)t * D, X + (size_t)t * D, m->attn_norm[l], D, 1e-5f);
        GEMM(&m->wq[l], Xn, Q);
        GEMM(&m->wk[l], Xn, K);
        GEMM(&m->wv[l], Xn, Vv);
        if (m->bias)
            for (int t = 0; t < n; t++) {
                addv(Q + (size_t)t * NQ, m->bq[l], NQ);
                addv(K + (size_t)t * NKV, m->bk[l], NKV);
                addv(Vv + (size_t)t * NKV, m->bv[l], NKV);
            }
        float* kcl = m->kc + (size_t)l * m->CTX * NKV;
        float* vcl = m->vc + (size_t)l * m->CTX * NKV;
        for (int t = 0; t < n; t++) {
            qk_norm(m, l, Q + (size_t)t * NQ, K + (size_t)t * NKV);
            orco_rope(Q + (size_t)t * NQ, K + (size_t)t * NKV, m->H, m->KVH, m->HD, sp + t, m->rope);
            memcpy(kcl + (size_t)(sp + t) * NKV, K + (size_t)t * NKV, sizeof(float) * NKV);
            memcpy(vcl + (size_t)(sp + t) * NKV, Vv + (size_t)t * NKV, sizeof(float) * NKV);
        }
        for (int t = 0; t < n; t++)
            orco_attention(Q + (size_t)t * NQ, kcl, vcl, m->H, m->KVH, m->HD, sp + t, AO + (size_t)t * NQ);
        GEMM(&m->wo[l], AO, XO);
        for (size_t i = 0; i < (size_t)n * D; i++) X[i] += XO[i];
        for (int t = 0; t < n; t++) orco_rmsnorm(Xn + (size_t)t * D, X + (size_t)t * D, m->ffn_norm[l], D, 1e-5f);
        GEMM(&m->wg[l], Xn, G);
        GEMM(&m->wu[l], Xn, U);
        for (size_t i = 0; i < (size_t)n * FF; i++) G[i] = (G[i] / (1.f + expf(-G[i]))) * U[i];
        GEMM(&m->wd[l], G, XO);
        for (size_t i = 0; i < (size_t)n * D; i++) X[i] += XO[i];
    }
    if (logits) {
        for (int t = 0; t < n; t++) orco_rmsnorm(Xn + (size_t)t * D, X + (size_t)t * D, m->out_norm, D, 1e-5f);
        GEMM(&m->head, Xn, logits);
        memcpy(m->x, Xn + (size_t)(n - 1) * D, sizeof(float) * D);
    }
#undef GEMM
    free(X); free(Xn); free(Q); free(K); free(Vv); free(AO); free(XO); free(G); free(U);
    return 0;
}

/* ── harness loops (bench_engine.cpp) ─────────────────────────────────────── */
int orco_greedy(orco_model* m, const int32_t* prompt, int np, int n_gen, int32_t* out) {
    orco_model_reset(m);
    orco_model_forward_batch(m, prompt, np - 1, 0, NULL);
    float* lg = (float*)malloc(sizeof(float) * (size_t)m->V);
    int32_t cur = prompt[np - 1];
    int pos = np - 1;
    for (int s = 0; s < n_gen; s++) {
        if (orco_model_forward(m, cur, pos++, lg)) { free(lg); return s; }
        out[s] = cur = orco_argmax(lg, m->V);
    }
    free(lg);
    return n_gen;
}

int orco_spec_greedy(orco_model* tg, orco_model* df, const int32_t* prompt, int np, int n_gen, int k, int32_t* out,
                     int64_t* st) {
    orco_model_reset(tg);
    orco_model_reset(df);
    orco_model_forward_batch(tg, prompt, np - 1, 0, NULL);
    orco_model_forward_batch(df, prompt, np - 1, 0, NULL);
    const int V = tg->V;
    float* blog = (float*)malloc(sizeof(float) * (size_t)(k + 1) * V);
    float* dl = (float*)malloc(sizeof(float) * (size_t)df->V);
    int pos = np - 1, ng = 0;
    int32_t next = prompt[np - 1];
    st[0] = st[1] = st[2] = 0;
    while (ng < n_gen && pos < tg->CTX - 1) {
        int32_t dtok[64], vin[65];
        int ndt = 0, dp = pos;
        int32_t dt = next;
        for (int i = 0; i < k && dp < df->CTX - 1; i++) {
            orco_model_forward(df, dt, dp++, dl);
            dtok[ndt++] = dt = orco_argmax(dl, df->V);
        }
        if (!ndt) break;
        st[1] += ndt;
        int nver = ndt + 1;
        if (pos + nver > tg->CTX) nver = tg->CTX - pos;
        vin[0] = next;
        for (int i = 0; i < nver - 1; i++) vin[i + 1] = dtok[i];
        orco_model_forward_batch(tg, vin, nver, pos, blog);
        st[2]++;
        int a = 0, brk = 0;
        for (int i = 0; i < ndt && i < nver; i++) {
            int32_t mt = orco_argmax(blog + (size_t)i * V, V);
            out[ng++] = mt;
            if (mt != dtok[i]) { next = mt; a = i; brk = 1; break; }
            st[0]++; a = i + 1; next = dtok[i];
            if (ng >= n_gen) { brk = 1; break; }
        }
        pos += a + 1;
        if (brk) continue;
        if (ng < n_gen && ndt < nver && pos < tg->CTX - 1) {
            out[ng++] = next = orco_argmax(blog + (size_t)ndt * V, V);
            orco_model_forward(df, dtok[ndt - 1], pos - 1, NULL);
        }
    }
    free(blog); free(dl);
    return ng;
}

/* ── std::mt19937 + Sampler (sampler.cpp) ─────────────────────────────────── */
struct orco_sampler {
    uint32_t mt[624]; int mti;
    float temp, top_p, pen; int top_k, last;
    int32_t* hist; int nh, cap;
};

static void mt_seed(orco_sampler* s, uint32_t seed) {
    s->mt[0] = seed;
    for (int i = 1; i < 624; i++) s->mt[i] = 1812433253u * (s->mt[i - 1] ^ (s->mt[i - 1] >> 30)) + (uint32_t)i;
    s->mti = 624;
}
uint32_t orco_mt_next(orco_sampler* s) {
    if (s->mti >= 624) {
        for (int i = 0; i < 624; i++) {
            uint32_t y = (s->mt[i] & 0x80000000u) | (s->mt[(i + 1) % 624] & 0x7FFFFFFFu);
            s->mt[i] = s->mt[(i + 397) % 624] ^ (y >> 1) ^ ((y & 1u) ? 0x9908B0DFu : 0u);
        }
        s->mti = 0;
    }
    uint32_t y = s->mt[s->mti++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9D2C5680u;
    y ^= (y << 15) & 0xEFC60000u;
    y ^= y >> 18;
    return y;
}
/* generate_canonical<float, 24>(mt19937) as libstdc++ computes it. */
static float mt_canonical(orco_sampler* s) {
    float r = (float)orco_mt_next(s) / 4294967296.0f;
    if (r >= 1.0f) r = nextafterf(1.0f, 0.0f);
    return r;
}

orco_sampler* orco_sampler_new(float temperature, float top_p, int top_k, float repeat_pen, int repeat_last,
                               uint64_t seed) {
    orco_sampler* s = (orco_sampler*)calloc(1, sizeof(orco_sampler));
    s->temp = temperature; s->top_p = top_p; s->top_k = top_k; s->pen = repeat_pen; s->last = repeat_last;
    s->cap = 2 * repeat_last + 16;
    s->hist = (int32_t*)calloc((size_t)s->cap, sizeof(int32_t));
    mt_seed(s, (uint32_t)seed);
    return s;
}
void orco_sampler_free(orco_sampler* s) { if (s) { free(s->hist); free(s); } }

void orco_sampler_record(orco_sampler* s, int32_t tok) { /* :99-105 */
    if (s->nh >= s->cap) { s->cap *= 2; s->hist = (int32_t*)realloc(s->hist, sizeof(int32_t) * (size_t)s->cap); }
    s->hist[s->nh++] = tok;
    if (s->nh > s->last * 2) {
        memmove(s->hist, s->hist + s->last, sizeof(int32_t) * (size_t)(s->nh - s->last));
        s->nh -= s->last;
    }
}
int orco_sampler_history(const orco_sampler* s, int32_t* out, int cap) {
    int n = s->nh < cap ? s->nh : cap;
    memcpy(out, s->hist + (s->nh - n), sizeof(int32_t) * (size_t)n);
    return n;
}

static void penalty(float* lg, int n, const int32_t* h, int nh, int last, float pen) { /* :15-27 */
    if (pen <= 1.f || nh == 0) return;
    int start = nh - last;
    if (start < 0) start = 0;
    for (int i = start; i < nh; i++) {
        int32_t id = h[i];
        if (id < 0 || id >= n) continue;
        if (lg[id] > 0.f) lg[id] /= pen;
        else lg[id] *= pen;
    }
}
static void temperature(float* lg, int n, float T) { /* :35-39 */
    if (T <= 0.f || T == 1.f) return;
    float inv = 1.f / T;
    for (int i = 0; i < n; i++) lg[i] *= inv;
}

static const float* g_cmp_p;
static int cmp_desc(const void* a, const void* b) {
    float pa = g_cmp_p[*(const int32_t*)a], pb = g_cmp_p[*(const int32_t*)b];
    if (pa > pb) return -1;
    if (pa < pb) return 1;
    return *(const int32_t*)a - *(const int32_t*)b;
}
/* indices of the k largest probabilities, descending, ties by lower index */
static void topk_idx(const float* p, int n, int k, int32_t* idx) {
    int32_t* all = (int32_t*)malloc(sizeof(int32_t) * (size_t)n);
    for (int i = 0; i < n; i++) all[i] = i;
    g_cmp_p = p;
    qsort(all, (size_t)n, sizeof(int32_t), cmp_desc);
    memcpy(idx, all, sizeof(int32_t) * (size_t)k);
    free(all);
}

int32_t orco_sampler_sample(orco_sampler* s, float* lg, int n) { /* :91-97, 48-86 */
    penalty(lg, n, s->hist, s->nh, s->last, s->pen);
    temperature(lg, n, s->temp);
    int32_t tok;
    if (s->temp <= 0.f) tok = orco_argmax(lg, n);
    else {
        orco_softmax(lg, n);
        int k = s->top_k > 0 ? (s->top_k < n ? s->top_k : n) : n;
        int32_t* idx = (int32_t*)malloc(sizeof(int32_t) * (size_t)k);
        topk_idx(lg, n, k, idx);
        float cum = 0.f;
        int cut = k;
        for (int i = 0; i < k; i++) { cum += lg[idx[i]]; if (cum >= s->top_p) { cut = i + 1; break; } }
        float total = 0.f;
        for (int i = 0; i < cut; i++) total += lg[idx[i]];
        float r = mt_canonical(s) * total;
        tok = idx[0];
        for (int i = 0; i < cut; i++) { r -= lg[idx[i]]; if (r <= 0.f) { tok = idx[i]; break; } }
        free(idx);
    }
    orco_sampler_record(s, tok);
    return tok;
}

int orco_spec_engine(orco_model* tg, orco_model* df, const int32_t* ids, int n_ids, int n_predict, int k,
                     orco_sampler* s, int32_t* out, int64_t* st) { /* engine.cpp:100-240 */
    orco_model_reset(tg);
    orco_model_reset(df);
    const int V = tg->V;
    float* lb = (float*)malloc(sizeof(float) * (size_t)V);
    float* dl = (float*)malloc(sizeof(float) * (size_t)df->V);
    int pos = 0, ng = 0;
    st[0] = st[1] = st[2] = 0;
    if (n_ids - 1 > 0) {
        orco_model_forward_batch(tg, ids, n_ids - 1, 0, NULL);
        for (int i = 0; i < n_ids - 1; i++) orco_sampler_record(s, ids[i]);
        pos = n_ids - 1;
        orco_model_forward_batch(df, ids, n_ids - 1, 0, NULL);
    }
    int32_t next = ids[n_ids - 1];
    for (int step = 0; step < n_predict && pos < tg->CTX - 1;) {
        int32_t dts[64];
        int nd = 0, dp = pos;
        int32_t dt = next;
        for (int i = 0; i < k && dp < df->CTX - 1; i++) {
            orco_model_forward(df, dt, dp++, dl);
            dts[nd++] = dt = orco_argmax(dl, df->V);
        }
        if (!nd) break;
        st[1] += nd;
        int done = 0, acc = 0;
        int32_t verify = next;
        for (int i = 0; i < nd; i++) {
            if (pos >= tg->CTX - 1) { done = 1; break; }
            orco_model_forward(tg, verify, pos++, lb);
            st[2]++;
            int32_t mt = orco_sampler_sample(s, lb, V);
            orco_sampler_record(s, mt);
            if (mt != dts[i]) { next = mt; out[ng++] = next; step++; break; }
            next = dts[i];
            acc++; st[0]++;
            out[ng++] = next;
            step++;
            if (step >= n_predict) { done = 1; break; }
            verify = next;
        }
        if (done) break;
        if (acc == nd && pos < tg->CTX - 1) {
            orco_model_forward(tg, next, pos++, lb);
            st[2]++;
            next = orco_sampler_sample(s, lb, V);
            orco_sampler_record(s, next);
            out[ng++] = next;
            step++;
            orco_model_forward(df, dts[nd - 1], pos - 1, NULL);
        }
    }
    free(lb); free(dl);
    return ng;
}

/* ── north-star stochastic acceptance (no reference counterpart) ──────────── */
int orco_transform_probs(const float* logits, int n, const int32_t* hist, int n_hist, float T, float top_p,
                         int top_k, float pen, float* p) {
    float* lg = (float*)malloc(sizeof(float) * (size_t)n);
    memcpy(lg, logits, sizeof(float) * (size_t)n);
    penalty(lg, n, hist, n_hist, n_hist, pen);
    if (T <= 0.f) { /* greedy: all mass on the argmax */
        int a = orco_argmax(lg, n);
        for (int i = 0; i < n; i++) p[i] = 0.f;
        p[a] = 1.f;
        free(lg);
        return 1;
    }
    temperature(lg, n, T);
    orco_softmax(lg, n);
    int k = top_k > 0 ? (top_k < n ? top_k : n) : n;
    int32_t* idx = (int32_t*)malloc(sizeof(int32_t) * (size_t)k);
    topk_idx(lg, n, k, idx);
    float cum = 0.f;
    int cut = k;
    for (int i = 0; i < k; i++) { cum += lg[idx[i]]; if (cum >= top_p) { cut = i + 1; break; } }
    float total = 0.f;
    for (int i = 0; i < cut; i++) total += lg[idx[i]];
    for (int i = 0; i < n; i++) p[i] = 0.f;
    for (int i = 0; i < cut; i++) p[idx[i]] = lg[idx[i]] / total;
    free(idx); free(lg);
    return cut;
}

int32_t orco_accept_resample(const float* p, const float* q, int n, int32_t x, float u_acc, float u_res,
                             int* accepted) {
    float qx = q[x], px = p[x];
    if (qx > 0.f && u_acc * qx < px) { *accepted = 1; return x; }
    *accepted = 0;
    double tot = 0.0;
    for (int i = 0; i < n; i++) { float r = p[i] - q[i]; if (r > 0.f) tot += r; }
    if (tot <= 0.0) return orco_argmax(p, n);
    double r = (double)u_res * tot;
    int last = -1;
    for (int i = 0; i < n; i++) {
        float d = p[i] - q[i];
        if (d <= 0.f) continue;
        last = i;
        r -= d;
        if (r <= 0.0) return i;
    }
    return last;
}

/* One draw from non-negative weights w with the uniform u: the first index
 * whose running sum (double) of the positive weights reaches u * total;
 * the last positive index if rounding leaves the sum short. */
int32_t orco_pick(const float* w, int n, float u) {
    double tot = 0.0;
    for (int i = 0; i < n; i++) if (w[i] > 0.f) tot += w[i];
    double r = (double)u * tot;
    int last = -1;
    for (int i = 0; i < n; i++) {
        if (!(w[i] > 0.f)) continue;
        last = i;
        r -= w[i];
        if (r <= 0.0) return i;
    }
    return last < 0 ? 0 : last;
}

int orco_accept_chain(orco_sampler* s, const float* p, const float* q, int n, const int32_t* x, int k, int max_emit,
                      int32_t* out, int* accepted, int* all) {
    int emitted = 0;
    *accepted = *all = 0;
    for (int i = 0; i <= k && emitted < max_emit; i++) {
        int32_t tok;
        int acc = 0;
        const float* pi = p + (size_t)i * n;
        if (i == k) {
            tok = orco_pick(pi, n, mt_canonical(s));
            *all = 1;
        } else {
            const float* qi = q + (size_t)i * n;
            const float ua = mt_canonical(s);
            if (qi[x[i]] > 0.f && ua * qi[x[i]] < pi[x[i]]) { tok = x[i]; acc = 1; }
            else tok = orco_accept_resample(pi, qi, n, x[i], 1.f, mt_canonical(s), &acc);
        }
        orco_sampler_record(s, tok);
        out[emitted++] = tok;
        if (i == k || !acc) break;
        ++*accepted;
    }
    return emitted;
}

/* penalty window: the last `last` entries of history + pending proposals */
static int window(const orco_sampler* s, const int32_t* pend, int npend, int32_t* win) {
    int L = s->nh + npend, st = L - s->last > 0 ? L - s->last : 0, n = 0;
    for (int i = st; i < L; i++) win[n++] = i < s->nh ? s->hist[i] : pend[i - s->nh];
    return n;
}

int orco_spec_sampled(orco_model* tg, orco_model* df, const int32_t* prompt, int np, int n_gen, int k,
                      orco_sampler* s, int32_t* out, int64_t* st) {
    orco_model_reset(tg);
    orco_model_reset(df);
    const int V = tg->V, CTX = tg->CTX < df->CTX ? tg->CTX : df->CTX;
    int pos = 0, ng = 0;
    st[0] = st[1] = st[2] = 0;
    if (np > 1) { /* prompt[0..np-2] prefilled and recorded, as engine.cpp:115-125 */
        orco_model_forward_batch(tg, prompt, np - 1, 0, NULL);
        orco_model_forward_batch(df, prompt, np - 1, 0, NULL);
        for (int i = 0; i < np - 1; i++) orco_sampler_record(s, prompt[i]);
        pos = np - 1;
    }
    int32_t next = prompt[np - 1];
    float* lg = (float*)malloc(sizeof(float) * (size_t)(k + 1) * V);
    float* p = (float*)malloc(sizeof(float) * (size_t)(k + 1) * V);
    float* q = (float*)malloc(sizeof(float) * (size_t)k * V);
    int32_t* win = (int32_t*)malloc(sizeof(int32_t) * (size_t)(s->last + 1));
    int32_t vin[65];
    while (ng < n_gen && pos + k + 1 <= CTX) {
        vin[0] = next;
        for (int i = 0; i < k; i++) { /* proposals x_i ~ q_i */
            orco_model_forward(df, vin[i], pos + i, lg);
            int nw = window(s, vin + 1, i, win);
            orco_transform_probs(lg, V, win, nw, s->temp, s->top_p, s->top_k, s->pen, q + (size_t)i * V);
            vin[i + 1] = orco_pick(q + (size_t)i * V, V, mt_canonical(s));
        }
        orco_model_forward_batch(tg, vin, k + 1, pos, lg);
        for (int r = 0; r <= k; r++) {
            int nw = window(s, vin + 1, r, win);
            orco_transform_probs(lg + (size_t)r * V, V, win, nw, s->temp, s->top_p, s->top_k, s->pen,
                                 p + (size_t)r * V);
        }
        st[1] += k;
        st[2]++;
        int acc = 0, all = 0;
        const int emitted = orco_accept_chain(s, p, q, V, vin + 1, k, n_gen - ng, out + ng, &acc, &all);
        st[0] += acc;
        ng += emitted;
        next = out[ng - 1];
        pos += emitted;
        if (all && ng < n_gen) orco_model_forward(df, vin[k], pos - 1, NULL); /* the draft lacks x_{k-1} */
    }
    free(lg); free(p); free(q); free(win);
    return ng;
}
