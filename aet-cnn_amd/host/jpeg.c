/*
 * jpeg.c -- a baseline / extended sequential JPEG decoder (ITU-T T.81) for
 * the input pipeline's image files.  The reference reads its image lists
 * with the vendored stb_image (NImage.loadImage, NImage.c:587-623), which
 * decodes JPEG among other formats; this is this build's own decoder of the
 * same published format, not a port of stb_image.
 *
 * Supported: 8-bit samples, Huffman coding, SOF0 / SOF1 frames, one or three
 * components (greyscale, YCbCr per JFIF, or RGB when an Adobe APP14 marker
 * says no transform), any sampling factors 1-4, interleaved and
 * non-interleaved scans, restart intervals.  Refused with a message:
 * progressive (SOF2) and arithmetic-coded frames, 12-bit samples, 2 or 4
 * components (CMYK / YCCK).
 *
 * Pipeline: entropy decoding into per-component coefficient blocks,
 * dequantisation, a separable floating-point 8x8 inverse DCT (T.81 A.3.3)
 * rounded to the nearest level and clamped to 0..255, 2x chroma upsampling
 * with the triangle ("fancy") filter -- each output sample is 3/4 of its
 * nearest input sample and 1/4 of the next one per doubled axis, edges
 * replicated -- and other ratios by replication, then the JFIF YCbCr -> RGB
 * conversion rounded to the nearest level.  Results agree with other
 * conforming decoders to within the rounding of the IDCT and the colour
 * conversion (about one level), not bit for bit.
 */
#include "jpeg.h"

#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* natural order of the k-th coefficient of the zig-zag sequence (T.81 A.3.6) */
static const unsigned char ZZ[64] = {
    0,  1,  8,  16, 9,  2,  3,  10, 17, 24, 32, 25, 18, 11, 4,  5,  12, 19, 26, 33, 40, 48,
    41, 34, 27, 20, 13, 6,  7,  14, 21, 28, 35, 42, 49, 56, 57, 50, 43, 36, 29, 22, 15, 23,
    30, 37, 44, 51, 58, 59, 52, 45, 38, 31, 39, 46, 53, 60, 61, 54, 47, 55, 62, 63};

typedef struct {
    int defined;
    int mincode[17], maxcode[18], valptr[17];
    unsigned char vals[256];
    uint16_t fast[1 << 9]; /* 9-bit prefix -> (length << 8) | value, 0: slow path */
} huff_t;

typedef struct {
    int id, h, v, tq;
    int bw, bh;      /* blocks per row / column, padded to whole MCUs */
    int xw, yh;      /* the component's own size in samples */
    int td, ta, dc;  /* the current scan's tables and DC predictor */
    int16_t *coef;   /* [bh][bw][64], natural order */
} comp_t;

typedef struct {
    const unsigned char *p, *end;
    uint32_t acc;
    int nbits;
    int marker; /* a marker met inside entropy-coded data (0: none) */
} bits_t;

typedef struct {
    uint16_t q[4][64]; /* natural order */
    int qdef[4];
    huff_t dc[4], ac[4];
    comp_t c[4];
    int nc, W, H, hmax, vmax, mcux, mcuy, restart;
    int frame, adobe, adobe_transform;
    const char *err;
} jpg_t;

static int bad(jpg_t *j, const char *why)
{
    if (!j->err) j->err = why;
    return -1;
}

static int u16(const unsigned char *p) { return (p[0] << 8) | p[1]; }

/* ---- Huffman tables (T.81 C, F.2.2.3) ------------------------------------- */
static int build_huff(huff_t *t, const unsigned char *counts, const unsigned char *vals, int n)
{
    memset(t, 0, sizeof(*t));
    memcpy(t->vals, vals, (size_t)n);
    int code = 0, k = 0;
    for (int len = 1; len <= 16; ++len) {
        t->valptr[len] = k;
        t->mincode[len] = code;
        code += counts[len - 1];
        k += counts[len - 1];
        if (code > (1 << len)) return -1; /* over-subscribed */
        t->maxcode[len] = counts[len - 1] ? code - 1 : -1;
        code <<= 1;
    }
    t->maxcode[17] = 0x7fffffff;
    /* fast table for codes of up to 9 bits */
    k = 0;
    code = 0;
    for (int len = 1; len <= 16; ++len) {
        for (int i = 0; i < counts[len - 1]; ++i, ++k, ++code) {
            if (len > 9) continue;
            const int shift = 9 - len, base = code << shift;
            for (int f = 0; f < (1 << shift); ++f)
                t->fast[base + f] = (uint16_t)((len << 8) | t->vals[k]);
        }
        code <<= 1;
    }
    t->defined = 1;
    return 0;
}

/* ---- bit reader over entropy-coded data with byte stuffing ---------------- */
static void fill(bits_t *b)
{
    while (b->nbits <= 24) {
        int c = 0;
        if (!b->marker && b->p < b->end) {
            c = *b->p;
            if (c == 0xff) {
                const int nx = b->p + 1 < b->end ? b->p[1] : 0xd9;
                if (nx == 0) {
                    b->p += 2; /* stuffed 0xff00 */
                } else {
                    b->marker = nx; /* stop before the marker; feed zeros */
                    c = 0;
                }
            } else {
                b->p++;
            }
        }
        b->acc |= (uint32_t)c << (24 - b->nbits);
        b->nbits += 8;
    }
}

static int decode_huff(bits_t *b, const huff_t *t)
{
    fill(b);
    const int f = t->fast[b->acc >> (32 - 9)];
    if (f) {
        const int len = f >> 8;
        b->acc <<= len;
        b->nbits -= len;
        return f & 255;
    }
    for (int len = 1; len <= 16; ++len) {
        const int code = (int)(b->acc >> (32 - len));
        if (code <= t->maxcode[len]) {
            b->acc <<= len;
            b->nbits -= len;
            return t->vals[t->valptr[len] + code - t->mincode[len]];
        }
    }
    return -1; /* no code of 16 bits or fewer matches */
}

/* RECEIVE and EXTEND (T.81 F.2.2.1): s bits as a signed difference */
static int receive_extend(bits_t *b, int s)
{
    if (s == 0) return 0;
    fill(b);
    const int v = (int)(b->acc >> (32 - s));
    b->acc <<= s;
    b->nbits -= s;
    return v < (1 << (s - 1)) ? v - (1 << s) + 1 : v;
}

static int decode_block(jpg_t *j, bits_t *b, comp_t *c, int16_t *blk)
{
    const int t = decode_huff(b, &j->dc[c->td]);
    if (t < 0 || t > 11) return bad(j, "corrupt DC code");
    c->dc += receive_extend(b, t);
    blk[0] = (int16_t)c->dc;
    for (int k = 1; k < 64;) {
        const int rs = decode_huff(b, &j->ac[c->ta]);
        if (rs < 0) return bad(j, "corrupt AC code");
        const int r = rs >> 4, s = rs & 15;
        if (s == 0) {
            if (r != 15) break; /* end of block */
            k += 16;
            continue;
        }
        k += r;
        if (k > 63) return bad(j, "AC run past the block");
        blk[ZZ[k]] = (int16_t)receive_extend(b, s);
        ++k;
    }
    return 0;
}

/* ---- one scan (T.81 B.2.3, F.1.1) ------------------------------------------ */
static int decode_scan(jpg_t *j, const unsigned char *seg, int seglen, const unsigned char **pp,
                       const unsigned char *end)
{
    const int ns = seg[0];
    if (ns < 1 || ns > j->nc || seglen < 1 + 2 * ns + 3) return bad(j, "bad SOS");
    comp_t *sc[4];
    for (int i = 0; i < ns; ++i) {
        const int id = seg[1 + 2 * i], tt = seg[2 + 2 * i];
        sc[i] = NULL;
        for (int k = 0; k < j->nc; ++k)
            if (j->c[k].id == id) sc[i] = &j->c[k];
        if (!sc[i]) return bad(j, "scan names an unknown component");
        sc[i]->td = tt >> 4;
        sc[i]->ta = tt & 15;
        if (sc[i]->td > 3 || sc[i]->ta > 3 || !j->dc[sc[i]->td].defined ||
            !j->ac[sc[i]->ta].defined)
            return bad(j, "scan uses an undefined Huffman table");
        sc[i]->dc = 0;
    }
    const int ss = seg[1 + 2 * ns], se = seg[2 + 2 * ns], ahl = seg[3 + 2 * ns];
    if (ss != 0 || se != 63 || ahl != 0) return bad(j, "not a sequential scan");
    bits_t b = {*pp, end, 0, 0, 0};
    int units_x, units_y;
    if (ns == 1) { /* non-interleaved: the component's own blocks */
        units_x = (sc[0]->xw + 7) / 8;
        units_y = (sc[0]->yh + 7) / 8;
    } else {
        units_x = j->mcux;
        units_y = j->mcuy;
    }
    const long total = (long)units_x * units_y;
    long todo = j->restart ? j->restart : total;
    for (long u = 0; u < total; ++u) {
        const int ux = (int)(u % units_x), uy = (int)(u / units_x);
        if (ns == 1) {
            comp_t *c = sc[0];
            if (decode_block(j, &b, c, c->coef + ((size_t)uy * c->bw + ux) * 64)) return -1;
        } else {
            for (int i = 0; i < ns; ++i) {
                comp_t *c = sc[i];
                for (int by = 0; by < c->v; ++by)
                    for (int bx = 0; bx < c->h; ++bx) {
                        const int x = ux * c->h + bx, y = uy * c->v + by;
                        if (decode_block(j, &b, c, c->coef + ((size_t)y * c->bw + x) * 64))
                            return -1;
                    }
            }
        }
        if (--todo == 0 && u + 1 < total) {
            /* restart interval: the bits left are padding; RSTn follows */
            while (b.p + 1 < b.end && !(b.p[0] == 0xff && b.p[1] != 0)) ++b.p;
            if (!(b.p + 1 < b.end && b.p[1] >= 0xd0 && b.p[1] <= 0xd7))
                return bad(j, "missing restart marker");
            b.p += 2;
            b.acc = 0;
            b.nbits = 0;
            b.marker = 0;
            for (int i = 0; i < ns; ++i) sc[i]->dc = 0;
            todo = j->restart;
        }
    }
    /* continue at the next marker */
    const unsigned char *p = b.p;
    while (p + 1 < end && !(p[0] == 0xff && p[1] != 0 && !(p[1] >= 0xd0 && p[1] <= 0xd7)))
        ++p;
    *pp = p;
    return 0;
}

/* ---- frame header (T.81 B.2.2) ---------------------------------------------- */
static int read_sof(jpg_t *j, const unsigned char *s, int len)
{
    if (len < 6) return bad(j, "bad SOF");
    if (s[0] != 8) return bad(j, "only 8-bit JPEG samples are supported");
    j->H = u16(s + 1);
    j->W = u16(s + 3);
    j->nc = s[5];
    if (j->W <= 0 || j->H <= 0) return bad(j, "bad JPEG size");
    if ((long)j->W * j->H > (1L << 28)) return bad(j, "JPEG too large");
    if (j->nc != 1 && j->nc != 3)
        return bad(j, "only 1- and 3-component JPEG is supported (not CMYK)");
    if (len < 6 + 3 * j->nc) return bad(j, "bad SOF");
    j->hmax = j->vmax = 1;
    for (int i = 0; i < j->nc; ++i) {
        comp_t *c = &j->c[i];
        c->id = s[6 + 3 * i];
        c->h = s[7 + 3 * i] >> 4;
        c->v = s[7 + 3 * i] & 15;
        c->tq = s[8 + 3 * i];
        if (c->h < 1 || c->h > 4 || c->v < 1 || c->v > 4 || c->tq > 3)
            return bad(j, "bad component in SOF");
        if (c->h > j->hmax) j->hmax = c->h;
        if (c->v > j->vmax) j->vmax = c->v;
    }
    j->mcux = (j->W + 8 * j->hmax - 1) / (8 * j->hmax);
    j->mcuy = (j->H + 8 * j->vmax - 1) / (8 * j->vmax);
    for (int i = 0; i < j->nc; ++i) {
        comp_t *c = &j->c[i];
        c->xw = (j->W * c->h + j->hmax - 1) / j->hmax;
        c->yh = (j->H * c->v + j->vmax - 1) / j->vmax;
        c->bw = j->mcux * c->h;
        c->bh = j->mcuy * c->v;
        c->coef = (int16_t *)calloc((size_t)c->bw * c->bh * 64, sizeof(int16_t));
        if (!c->coef) return bad(j, "out of memory");
    }
    j->frame = 1;
    return 0;
}

/* ---- sample reconstruction ---------------------------------------------------- */

/* C(u)/2 * cos((2x+1) u pi / 16), set once for every decoding thread */
/* cst[u][x] = C(u)/2 * cos((2x+1) u pi / 16), x fastest */
static float cst[8][8];
static pthread_once_t cs_once = PTHREAD_ONCE_INIT;
static void cs_init(void)
{
    for (int u = 0; u < 8; ++u)
        for (int x = 0; x < 8; ++x)
            cst[u][x] = (float)((u == 0 ? sqrt(0.5) : 1.0) * 0.5 * cos((2 * x + 1) * u * M_PI / 16));
}

/* the nearest level (halves up), clamped to 0..255: for v in (0, 255)
 * truncating v + 0.5 is floor(v + 0.5) */
static inline uint8_t clamp255f(float v)
{
    return v <= 0.f ? 0 : (v >= 255.f ? 255 : (uint8_t)(int)(v + 0.5f));
}

/* dequantised block -> 8x8 samples (T.81 A.3.3, separable, in float; rows
 * whose AC coefficients are all zero take their constant directly, which
 * most rows of a quantised block are) */
static void idct8x8(const int16_t *blk, const uint16_t *q, uint8_t *out, int stride)
{
    float t[8][8], o[8];
    /* rows: t[v][x] = sum_u cst[u][x] F[v][u], over the nonzero F only */
    for (int v = 0; v < 8; ++v) {
        for (int x = 0; x < 8; ++x) t[v][x] = 0.f;
        for (int u = 0; u < 8; ++u) {
            const int c = blk[v * 8 + u];
            if (!c) continue;
            const float fu = (float)c * q[v * 8 + u];
            for (int x = 0; x < 8; ++x) t[v][x] += cst[u][x] * fu;
        }
    }
    /* columns: out[y][x] = sum_v cst[v][y] t[v][x] */
    for (int y = 0; y < 8; ++y) {
        for (int x = 0; x < 8; ++x) o[x] = 128.f;
        for (int v = 0; v < 8; ++v) {
            const float cv = cst[v][y];
            for (int x = 0; x < 8; ++x) o[x] += cv * t[v][x];
        }
        for (int x = 0; x < 8; ++x) out[y * stride + x] = clamp255f(o[x]);
    }
}

/* a component's samples at its own resolution: [bh*8][bw*8] */
static uint8_t *component_plane(jpg_t *j, comp_t *c)
{
    pthread_once(&cs_once, cs_init);
    const int pw = c->bw * 8;
    uint8_t *pl = (uint8_t *)malloc((size_t)pw * c->bh * 8);
    if (!pl) return NULL;
    if (!j->qdef[c->tq]) {
        free(pl);
        return NULL;
    }
    for (int by = 0; by < c->bh; ++by)
        for (int bx = 0; bx < c->bw; ++bx)
            idct8x8(c->coef + ((size_t)by * c->bw + bx) * 64, j->q[c->tq],
                    pl + (size_t)by * 8 * pw + bx * 8, pw);
    return pl;
}

/* the component resampled to W x H (full resolution), 0..255 */
static uint8_t *upsample(jpg_t *j, comp_t *c, const uint8_t *pl)
{
    const int W = j->W, H = j->H, pw = c->bw * 8;
    uint8_t *out = (uint8_t *)malloc((size_t)W * H);
    if (!out) return NULL;
    const int fx = j->hmax / c->h, fy = j->vmax / c->v;
    const int exact = j->hmax % c->h == 0 && j->vmax % c->v == 0;
    if (fx == 1 && fy == 1 && exact) {
        for (int y = 0; y < H; ++y) memcpy(out + (size_t)y * W, pl + (size_t)y * pw, (size_t)W);
        return out;
    }
    if (exact && fx <= 2 && fy <= 2) {
        /* triangle filter per doubled axis (the nearer input sample weighs
         * 3/4, the next one 1/4, edges repeat): one output row at a time, the
         * vertical pass first; the integer sums carry 4 (one axis) or 16
         * (both) times the sample and are rounded half up once at the end */
        const int cw = c->xw, ch = c->yh, ow = cw * fx, oh = ch * fy;
        int *v = (int *)malloc(sizeof(int) * (size_t)cw);
        int *h = (int *)malloc(sizeof(int) * (size_t)ow);
        if (!v || !h) {
            free(v);
            free(h);
            free(out);
            return NULL;
        }
        const int sh = 2 * (fx - 1) + 2 * (fy - 1), half = sh ? 1 << (sh - 1) : 0;
        const int wn = W < ow ? W : ow;
        for (int y = 0; y < H; ++y) {
            const int oy = y < oh ? y : oh - 1;
            if (fy == 2) {
                const int i = oy >> 1,
                          k = (oy & 1) ? (i + 1 < ch ? i + 1 : ch - 1) : (i > 0 ? i - 1 : 0);
                const uint8_t *r0 = pl + (size_t)i * pw, *r1 = pl + (size_t)k * pw;
                for (int x = 0; x < cw; ++x) v[x] = 3 * r0[x] + r1[x];
            } else {
                const uint8_t *r0 = pl + (size_t)oy * pw;
                for (int x = 0; x < cw; ++x) v[x] = r0[x];
            }
            if (fx == 2) {
                for (int x = 0; x < cw; ++x) {
                    const int l = v[x > 0 ? x - 1 : 0], r = v[x + 1 < cw ? x + 1 : cw - 1];
                    h[2 * x] = 3 * v[x] + l;
                    h[2 * x + 1] = 3 * v[x] + r;
                }
            } else {
                memcpy(h, v, sizeof(int) * (size_t)cw);
            }
            uint8_t *o = out + (size_t)y * W; /* the sums stay <= 255 after the shift */
            for (int x = 0; x < wn; ++x) o[x] = (uint8_t)((h[x] + half) >> sh);
            for (int x = wn; x < W; ++x) o[x] = o[wn - 1];
        }
        free(v);
        free(h);
        return out;
    }
    /* other ratios: nearest sample (replication) */
    for (int y = 0; y < H; ++y) {
        const int sy = (int)((long)y * c->v / j->vmax);
        for (int x = 0; x < W; ++x) {
            const int sx = (int)((long)x * c->h / j->hmax);
            out[(size_t)y * W + x] = pl[(size_t)sy * pw + sx];
        }
    }
    return out;
}

int an_jpeg_decode(const unsigned char *buf, size_t len, int *Wp, int *Hp, int *chans,
                   unsigned char **px, const char **why)
{
    jpg_t *j = (jpg_t *)calloc(1, sizeof(jpg_t));
    if (!j) {
        *why = "out of memory";
        return -1;
    }
    const unsigned char *p = buf, *end = buf + len;
    int rc = 0, scans = 0;
    if (len < 4 || p[0] != 0xff || p[1] != 0xd8) rc = bad(j, "not a JPEG file");
    p += 2;
    while (!rc) {
        /* the next marker (fill bytes 0xff allowed) */
        while (p < end && *p != 0xff) ++p;
        while (p < end && *p == 0xff) ++p;
        if (p >= end) {
            rc = bad(j, "truncated JPEG");
            break;
        }
        const int m = *p++;
        if (m == 0xd9) break; /* EOI */
        if (m >= 0xd0 && m <= 0xd7) continue;
        if (p + 2 > end) {
            rc = bad(j, "truncated JPEG");
            break;
        }
        const int L = u16(p);
        if (L < 2 || p + L > end) {
            rc = bad(j, "truncated JPEG segment");
            break;
        }
        const unsigned char *s = p + 2;
        const int sl = L - 2;
        p += L;
        switch (m) {
        case 0xc0:
        case 0xc1:
            if (j->frame) rc = bad(j, "two frames");
            else rc = read_sof(j, s, sl);
            break;
        case 0xc2:
        case 0xc6:
        case 0xca:
        case 0xce:
            rc = bad(j, "progressive JPEG is not supported");
            break;
        case 0xc3:
        case 0xc5:
        case 0xc7:
        case 0xcb:
        case 0xcd:
        case 0xcf:
            rc = bad(j, "lossless / hierarchical JPEG is not supported");
            break;
        case 0xc9:
            rc = bad(j, "arithmetic-coded JPEG is not supported");
            break;
        case 0xc4: { /* DHT: one or more tables */
            int o = 0;
            while (!rc && o < sl) {
                if (o + 17 > sl) {
                    rc = bad(j, "bad DHT");
                    break;
                }
                const int tc = s[o] >> 4, th = s[o] & 15;
                int n = 0;
                for (int i = 0; i < 16; ++i) n += s[o + 1 + i];
                if (tc > 1 || th > 3 || n > 256 || o + 17 + n > sl) {
                    rc = bad(j, "bad DHT");
                    break;
                }
                huff_t *t = tc ? &j->ac[th] : &j->dc[th];
                if (build_huff(t, s + o + 1, s + o + 17, n)) rc = bad(j, "bad Huffman table");
                o += 17 + n;
            }
            break;
        }
        case 0xdb: { /* DQT */
            int o = 0;
            while (!rc && o < sl) {
                const int pq = s[o] >> 4, tq = s[o] & 15, sz = pq ? 128 : 64;
                if (pq > 1 || tq > 3 || o + 1 + sz > sl) {
                    rc = bad(j, "bad DQT");
                    break;
                }
                for (int k = 0; k < 64; ++k)
                    j->q[tq][ZZ[k]] = (uint16_t)(pq ? u16(s + o + 1 + 2 * k) : s[o + 1 + k]);
                j->qdef[tq] = 1;
                o += 1 + sz;
            }
            break;
        }
        case 0xdd: /* DRI */
            if (sl < 2) rc = bad(j, "bad DRI");
            else j->restart = u16(s);
            break;
        case 0xee: /* APP14 "Adobe": colour transform flag */
            if (sl >= 12 && !memcmp(s, "Adobe", 5)) {
                j->adobe = 1;
                j->adobe_transform = s[11];
            }
            break;
        case 0xda: /* SOS, then the entropy-coded segment */
            if (!j->frame) rc = bad(j, "scan before the frame header");
            else {
                rc = decode_scan(j, s, sl, &p, end);
                ++scans;
            }
            break;
        default: /* APPn, COM and the rest: skipped */
            break;
        }
    }
    uint8_t *rgb = NULL;
    if (!rc && !scans) rc = bad(j, "no image data");
    if (!rc) {
        uint8_t *full[3] = {NULL, NULL, NULL};
        for (int i = 0; i < j->nc && !rc; ++i) {
            uint8_t *pl = component_plane(j, &j->c[i]);
            if (!pl) {
                rc = bad(j, j->qdef[j->c[i].tq] ? "out of memory" : "undefined quantisation table");
                break;
            }
            full[i] = upsample(j, &j->c[i], pl);
            free(pl);
            if (!full[i]) rc = bad(j, "out of memory");
        }
        const size_t np = (size_t)j->W * j->H;
        if (!rc) rgb = (uint8_t *)malloc(np * (size_t)j->nc);
        if (!rc && !rgb) rc = bad(j, "out of memory");
        if (!rc && j->nc == 1) memcpy(rgb, full[0], np);
        if (!rc && j->nc == 3) {
            /* RGB components: an Adobe marker with transform 0, or ids
             * 'R', 'G', 'B'; otherwise YCbCr (JFIF) */
            const int is_rgb = (j->adobe && j->adobe_transform == 0) ||
                               (j->c[0].id == 'R' && j->c[1].id == 'G' && j->c[2].id == 'B');
            for (size_t i = 0; i < np; ++i) {
                if (is_rgb) {
                    rgb[3 * i] = full[0][i];
                    rgb[3 * i + 1] = full[1][i];
                    rgb[3 * i + 2] = full[2][i];
                    continue;
                }
                const float y = full[0][i], cb = full[1][i] - 128.f, cr = full[2][i] - 128.f;
                rgb[3 * i] = clamp255f(y + 1.402f * cr);
                rgb[3 * i + 1] = clamp255f(y - 0.344136f * cb - 0.714136f * cr);
                rgb[3 * i + 2] = clamp255f(y + 1.772f * cb);
            }
        }
        for (int i = 0; i < 3; ++i) free(full[i]);
    }
    for (int i = 0; i < 4; ++i) free(j->c[i].coef);
    if (rc) {
        free(rgb);
        *why = j->err ? j->err : "corrupt JPEG";
        free(j);
        return -1;
    }
    *Wp = j->W;
    *Hp = j->H;
    *chans = j->nc;
    *px = rgb;
    free(j);
    return 0;
}
