/*
 * pkv_oracle.c -- CPU restatement of mlx-one's paged KV arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Loaded (through oracle/cport.py) by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the checker and
 * the timed CPU baseline; never linked into or called by the product library.
 *
 * Page format is the reference's own (src/mlx_one/engine/paged_attention.py:31-35):
 * per page, K codes [HK][P][Dq] u8, K scale [HK][P][NG] f16, K bias (same),
 * then the same three tensors for V; Dq = Dp for 8 bit and Dp/2 for 4 bit,
 * Dp = ceil(D/G)*G, NG = Dp/G.  Float pages hold K [HK][P][D] and V in
 * bf16 or f16 bits.
 *
 * Functions and what pins them:
 *   pkvo_f32_to_f16      IEEE round-to-nearest-even, checked against numpy's
 *                        float16 cast on every sign/exponent and tie pattern.
 *   pkvo_quantize_rows   paged.py:24-41, checked bit-exact against the numpy
 *                        restatement, which is checked against golden vectors
 *                        written by the reference's own quantize_page.
 *   pkvo_paged_attention paged_attention.py:209-246 semantics (causal by
 *                        position, GQA kh = h / (H/HK), padded query rows 0,
 *                        normaliser floored at 1e-20), checked against the
 *                        numpy oracle on seeded inputs.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- scalar formats --------------------------------------------------- */

uint16_t pkvo_f32_to_f16(float value)
{
    uint32_t x;
    memcpy(&x, &value, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (exp == 0xFFu)                                  /* inf / nan */
        return (uint16_t)(sign | 0x7C00u | (man ? 0x200u | (man >> 13) : 0u));
    int e = (int)exp - 127 + 15;                       /* rebias */
    if (e >= 31)                                       /* overflow -> inf */
        return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {                                      /* f16 subnormal or zero */
        if (e < -10)
            return (uint16_t)sign;
        uint32_t full = man | 0x800000u;               /* 24-bit significand */
        int shift = 14 - e;                            /* keep 10 - (1 - e) bits */
        uint32_t kept = full >> shift;
        uint32_t rest = full & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rest > half || (rest == half && (kept & 1u)))
            kept += 1u;                                /* may carry into exp 1 */
        return (uint16_t)(sign | kept);
    }
    uint32_t kept = man >> 13;
    uint32_t rest = man & 0x1FFFu;
    uint32_t out = ((uint32_t)e << 10) | kept;
    if (rest > 0x1000u || (rest == 0x1000u && (kept & 1u)))
        out += 1u;                                     /* carry may reach inf */
    return (uint16_t)(sign | out);
}

float pkvo_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t x;
    if (exp == 0) {
        if (man == 0) {
            x = sign;
        } else {                                       /* normalise subnormal */
            int e = -1;
            do { man <<= 1; e++; } while (!(man & 0x400u));
            x = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3FFu) << 13);
        }
    } else if (exp == 31) {
        x = sign | 0x7F800000u | (man << 13);
    } else {
        x = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

static inline float bf16_to_f32(uint16_t h)
{
    uint32_t x = (uint32_t)h << 16;
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* ---- quantizer: paged.py:24-41 --------------------------------------- */

/*
 * x: rows x dim float32 values (f16- or bf16-valued).  Outputs in the
 * reference format: codes rows x (Dp*bits/8), scale/bias rows x NG (f16 bits).
 */
void pkvo_quantize_rows(const float *x, int64_t rows, int dim, int bits, int group,
                        uint8_t *codes, uint16_t *scale, uint16_t *bias)
{
    int padded = (dim + group - 1) / group * group;
    int ngroups = padded / group;
    int levels = (1 << bits) - 1;
    int bytes = bits == 4 ? padded / 2 : padded;
#ifdef _OPENMP
#pragma omp parallel
#endif
    {
    float *row = (float *)malloc(sizeof(float) * (size_t)padded);
    uint8_t *code = (uint8_t *)malloc((size_t)padded);
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
    for (int64_t r = 0; r < rows; ++r) {
        const float *src = x + r * dim;
        for (int d = 0; d < padded; ++d)
            row[d] = d < dim ? src[d] : 0.0f;            /* mx.pad with zeros */
        for (int g = 0; g < ngroups; ++g) {
            const float *v = row + g * group;
            float lo = v[0], hi = v[0];
            for (int i = 1; i < group; ++i) {
                lo = v[i] < lo ? v[i] : lo;
                hi = v[i] > hi ? v[i] : hi;
            }
            uint16_t b16 = pkvo_f32_to_f16(lo);          /* bias rounded first */
            float b = pkvo_f16_to_f32(b16);
            float s = (hi - b) / (float)levels;          /* f32 IEEE division */
            s = s > 1e-6f ? s : 1e-6f;                   /* maximum(., 1e-6) */
            uint16_t s16 = pkvo_f32_to_f16(s);
            float sf = pkvo_f16_to_f32(s16);
            scale[r * ngroups + g] = s16;
            bias[r * ngroups + g] = b16;
            for (int i = 0; i < group; ++i) {
                float c = rintf((v[i] - b) / sf);        /* half to even */
                c = c < 0.0f ? 0.0f : (c > (float)levels ? (float)levels : c);
                code[g * group + i] = (uint8_t)c;
            }
        }
        uint8_t *dst = codes + r * bytes;
        if (bits == 8) {
            memcpy(dst, code, (size_t)padded);
        } else {
            for (int i = 0; i < padded / 2; ++i)
                dst[i] = (uint8_t)(code[2 * i] | (code[2 * i + 1] << 4));
        }
    }
    free(row);
    free(code);
    }
}

/* ---- paged attention: paged_attention.py:209-246 --------------------- */

typedef struct {
    int hk, page, dim, bits, group, padded, ngroups, qbytes, float_f16;
    const uint8_t *kc, *vc;
    const uint16_t *ks, *kb, *vs, *vb;     /* quantized metadata (f16 bits) */
    const uint16_t *kf, *vf;               /* float pages */
} pages_t;

/* Dequantize (or widen) K and V of token slot `t` of page `page`, head `kh`. */
static void load_token(const pages_t *p, int64_t page, int kh, int t, float *k, float *v)
{
    if (p->bits == 0) {
        size_t base = (((size_t)page * p->hk + kh) * p->page + t) * p->dim;
        for (int d = 0; d < p->dim; ++d) {
            k[d] = p->float_f16 ? pkvo_f16_to_f32(p->kf[base + d]) : bf16_to_f32(p->kf[base + d]);
            v[d] = p->float_f16 ? pkvo_f16_to_f32(p->vf[base + d]) : bf16_to_f32(p->vf[base + d]);
        }
        return;
    }
    size_t row = ((size_t)page * p->hk + kh) * p->page + t;
    const uint8_t *kc = p->kc + row * p->qbytes, *vc = p->vc + row * p->qbytes;
    const uint16_t *ks = p->ks + row * p->ngroups, *kb = p->kb + row * p->ngroups;
    const uint16_t *vs = p->vs + row * p->ngroups, *vb = p->vb + row * p->ngroups;
    for (int d = 0; d < p->dim; ++d) {
        int ck, cv;
        if (p->bits == 4) {
            ck = (kc[d / 2] >> ((d % 2) * 4)) & 15;
            cv = (vc[d / 2] >> ((d % 2) * 4)) & 15;
        } else {
            ck = kc[d];
            cv = vc[d];
        }
        int g = d / p->group;
        k[d] = (float)ck * pkvo_f16_to_f32(ks[g]) + pkvo_f16_to_f32(kb[g]);
        v[d] = (float)cv * pkvo_f16_to_f32(vs[g]) + pkvo_f16_to_f32(vb[g]);
    }
}

/*
 * q: [B][H][Q][D] float32.  block_table: [B][max_pages] page ids.
 * lengths[b]: tokens in the cache; positions[b*Q+qi]: logical query position;
 * widths[b]: real query rows.  out: [B][H][Q][D] float32, padded rows zero.
 * threads <= 0 uses the OpenMP default.  Returns 0.
 */
int pkvo_paged_attention(const float *q, int B, int H, int HK, int Q, int D, int P,
                         int bits, int group, int float_f16,
                         const int32_t *block_table, int max_pages,
                         const int32_t *lengths, const int32_t *positions,
                         const int32_t *widths,
                         const uint8_t *kc, const uint16_t *ks, const uint16_t *kb,
                         const uint8_t *vc, const uint16_t *vs, const uint16_t *vb,
                         const uint16_t *kf, const uint16_t *vf,
                         float scale, float *out, int threads)
{
    pages_t p;
    p.hk = HK; p.page = P; p.dim = D; p.bits = bits; p.group = group > 0 ? group : 32;
    p.padded = (D + p.group - 1) / p.group * p.group;
    p.ngroups = p.padded / p.group;
    p.qbytes = bits == 4 ? p.padded / 2 : p.padded;
    p.float_f16 = float_f16;
    p.kc = kc; p.vc = vc; p.ks = ks; p.kb = kb; p.vs = vs; p.vb = vb; p.kf = kf; p.vf = vf;
    int group_heads = H / HK;
    int rows = group_heads * Q;
    memset(out, 0, sizeof(float) * (size_t)B * H * Q * D);
#ifdef _OPENMP
    if (threads > 0)
        omp_set_num_threads(threads);
#pragma omp parallel
#endif
    {
        int longest = 0;
        for (int b = 0; b < B; ++b)
            longest = lengths[b] > longest ? lengths[b] : longest;
        float *kbuf = (float *)malloc(sizeof(float) * (size_t)D);
        float *vbuf = (float *)malloc(sizeof(float) * (size_t)D);
        float *scores = (float *)malloc(sizeof(float) * (size_t)rows * (longest + 1));
        double *acc = (double *)malloc(sizeof(double) * (size_t)rows * D);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (int job = 0; job < B * HK; ++job) {
            int b = job / HK, kh = job % HK;
            int length = lengths[b];
            /* pass 1: scores of every (query, head) row of this KV head */
            for (int t = 0; t < length; ++t) {
                int64_t page = block_table[(size_t)b * max_pages + t / P];
                load_token(&p, page, kh, t % P, kbuf, vbuf);
                for (int r = 0; r < rows; ++r) {
                    int qi = r / group_heads, h = kh * group_heads + r % group_heads;
                    const float *qv = q + (((size_t)b * H + h) * Q + qi) * D;
                    float dot = 0.0f;
                    for (int d = 0; d < D; ++d)
                        dot += qv[d] * kbuf[d];
                    int visible = qi < widths[b] && t <= positions[(size_t)b * Q + qi];
                    scores[(size_t)r * length + t] = visible ? dot * scale : -INFINITY;
                }
            }
            /* softmax per row */
            for (int r = 0; r < rows; ++r) {
                float *s = scores + (size_t)r * length;
                float top = -INFINITY;
                for (int t = 0; t < length; ++t)
                    top = s[t] > top ? s[t] : top;
                for (int t = 0; t < length; ++t)
                    s[t] = top == -INFINITY ? 0.0f : expf(s[t] - top);
            }
            /* pass 2: weighted V */
            memset(acc, 0, sizeof(double) * (size_t)rows * D);
            double *norm = (double *)calloc((size_t)rows, sizeof(double));
            for (int t = 0; t < length; ++t) {
                int64_t page = block_table[(size_t)b * max_pages + t / P];
                load_token(&p, page, kh, t % P, kbuf, vbuf);
                for (int r = 0; r < rows; ++r) {
                    float w = scores[(size_t)r * length + t];
                    if (w == 0.0f)
                        continue;
                    norm[r] += w;
                    double *a = acc + (size_t)r * D;
                    for (int d = 0; d < D; ++d)
                        a[d] += (double)w * vbuf[d];
                }
            }
            for (int r = 0; r < rows; ++r) {
                int qi = r / group_heads, h = kh * group_heads + r % group_heads;
                if (qi >= widths[b])
                    continue;
                double n = norm[r] > 1e-20 ? norm[r] : 1e-20;
                float *o = out + (((size_t)b * H + h) * Q + qi) * D;
                for (int d = 0; d < D; ++d)
                    o[d] = (float)(acc[(size_t)r * D + d] / n);
            }
            free(norm);
        }
        free(kbuf);
        free(vbuf);
        free(scores);
        free(acc);
    }
    return 0;
}

int pkvo_version(void) { return 1; }
