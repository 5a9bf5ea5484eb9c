/*
 * image.c -- the images of the input pipeline: file decoding and the
 * training-time augmentation of one image.  Reference behaviour replaced
 * (paths under /root/reference/src/com/ai/dnn/):
 *
 *   NImage.reload            NImage.c:638-658   file -> planar float / 255,
 *                                               size and channels must match
 *   NImage.randomAugment     NImage.c:1016-1034 random aspect, crop size,
 *                                               rotation and offset
 *   NImage.rotateCrop        NImage.c:551-572   bilinear resampling
 *   NImage.bilinearInterpolate / getPixelExtend NImage.c:138-158
 *   NImage.flip              NImage.c:355-370
 *   NImage.randomDistort / distort / rgbToHsv / hsvToRgb / scaleChannel /
 *   constrainImage           NImage.c:201-352
 *   NImage.resizeImage       NImage.c:474-530
 *   DnnUtils.randScale / randUniform / randInt / randUniformStrong
 *                            DnnUtils.c:188-232, DnnUtils.h:75-101
 *   ImageData.loadImageAugmentPaths ImageData.c:56-73 (the order of the steps)
 *   ImageData.fillTruthSmooth       ImageData.c:80-104 (labels from paths)
 *
 * The reference decodes files with the vendored stb_image; this file has its
 * own decoders for PNG (8-bit, non-interlaced, every colour type; zlib's
 * inflate) and binary PPM / PGM, and host/jpeg.c one for baseline /
 * extended sequential JPEG.  The reference's random numbers come from
 * the shared rand() stream; here every draw of image i of batch k is a
 * counter-based hash (an_feeder_sample) with its own salt, fed through the
 * reference's formulas with RAND_MAX = 2^31 - 1, so an image's augmentation
 * does not depend on the threads that load it.
 */
#include "aetcnn_net.h"
#include "jpeg.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <zlib.h>

/* ---- decoding -------------------------------------------------------------- */
static int fail(const char *path, const char *why)
{
    fprintf(stderr, "an_image_load: %s: %s\n", path, why);
    return ACH_EINVAL;
}

static uint32_t be32(const unsigned char *p)
{
    return ((uint32_t)p[0] << 24) | ((uint32_t)p[1] << 16) | ((uint32_t)p[2] << 8) | p[3];
}

static unsigned char *read_file(const char *path, size_t *len)
{
    FILE *f = fopen(path, "rb");
    if (!f) return NULL;
    unsigned char *buf = NULL;
    size_t cap = 0, n = 0;
    for (;;) {
        if (n == cap) {
            cap = cap ? 2 * cap : 1 << 16;
            unsigned char *nb = (unsigned char *)realloc(buf, cap);
            if (!nb) {
                free(buf);
                fclose(f);
                return NULL;
            }
            buf = nb;
        }
        const size_t got = fread(buf + n, 1, cap - n, f);
        n += got;
        if (got == 0) break;
    }
    fclose(f);
    *len = n;
    return buf;
}

static int paeth(int a, int b, int c)
{
    const int p = a + b - c, pa = abs(p - a), pb = abs(p - b), pc = abs(p - c);
    if (pa <= pb && pa <= pc) return a;
    return pb <= pc ? b : c;
}

/* PNG (ISO/IEC 15948): 8-bit samples, no interlace.  Native channels:
 * grey 1, RGB 3, palette 3 (4 with a tRNS chunk), grey+alpha 2, RGBA 4.
 * *px: W*H*chans interleaved 8-bit samples (malloc'd).                     */
static int decode_png(const char *path, const unsigned char *buf, size_t len, int *Wp, int *Hp,
                      int *chansp, unsigned char **px)
{
    static const unsigned char sig[8] = {137, 80, 78, 71, 13, 10, 26, 10};
    if (len < 8 || memcmp(buf, sig, 8)) return fail(path, "not a PNG file");
    size_t pos = 8;
    int W = 0, H = 0, depth = 0, ctype = -1, interlace = 0, npal = 0, has_trns = 0;
    unsigned char pal[256][4];
    unsigned char *idat = NULL;
    size_t nidat = 0;
    int rc = ACH_OK;
    while (pos + 12 <= len) {
        const uint32_t clen = be32(buf + pos);
        const unsigned char *type = buf + pos + 4, *data = buf + pos + 8;
        if (clen > len - pos - 12) {
            rc = fail(path, "truncated chunk");
            break;
        }
        if (!memcmp(type, "IHDR", 4) && clen >= 13) {
            W = (int)be32(data);
            H = (int)be32(data + 4);
            depth = data[8];
            ctype = data[9];
            interlace = data[12];
        } else if (!memcmp(type, "PLTE", 4)) {
            npal = (int)(clen / 3);
            if (npal > 256) npal = 256;
            for (int i = 0; i < npal; ++i) {
                pal[i][0] = data[3 * i];
                pal[i][1] = data[3 * i + 1];
                pal[i][2] = data[3 * i + 2];
                pal[i][3] = 255;
            }
        } else if (!memcmp(type, "tRNS", 4) && ctype == 3) {
            has_trns = 1;
            for (uint32_t i = 0; i < clen && (int)i < npal; ++i) pal[i][3] = data[i];
        } else if (!memcmp(type, "IDAT", 4)) {
            unsigned char *ni = (unsigned char *)realloc(idat, nidat + clen + 1);
            if (!ni) {
                rc = fail(path, "out of host memory");
                break;
            }
            idat = ni;
            memcpy(idat + nidat, data, clen);
            nidat += clen;
        } else if (!memcmp(type, "IEND", 4)) {
            break;
        }
        pos += 12 + clen;
    }
    int chans = 0;
    if (rc == ACH_OK) {
        switch (ctype) {
        case 0: chans = 1; break;
        case 2: chans = 3; break;
        case 3: chans = has_trns ? 4 : 3; break;
        case 4: chans = 2; break;
        case 6: chans = 4; break;
        default: rc = fail(path, "missing or unknown IHDR colour type");
        }
    }
    if (rc == ACH_OK && (depth != 8 || interlace != 0))
        rc = fail(path, "only 8-bit non-interlaced PNG is supported");
    if (rc == ACH_OK && (W <= 0 || H <= 0 || W > (1 << 15) || H > (1 << 15)))
        rc = fail(path, "image size out of range");
    if (rc == ACH_OK && !idat) rc = fail(path, "no image data");
    const int spp = ctype == 3 ? 1 : chans; /* bytes per pixel in the stream */
    const size_t stride = (size_t)W * spp;
    unsigned char *raw = NULL;
    if (rc == ACH_OK) {
        uLongf rawlen = (uLongf)((stride + 1) * (size_t)H);
        raw = (unsigned char *)malloc(rawlen);
        if (!raw) rc = fail(path, "out of host memory");
        else if (uncompress(raw, &rawlen, idat, (uLong)nidat) != Z_OK ||
                 rawlen != (uLongf)((stride + 1) * (size_t)H))
            rc = fail(path, "corrupt image data");
    }
    if (rc == ACH_OK) {
        /* undo the per-row filters in place (prior row already decoded) */
        for (int y = 0; y < H && rc == ACH_OK; ++y) {
            unsigned char *row = raw + (size_t)y * (stride + 1);
            const int ft = row[0];
            if (ft > 4) {
                rc = fail(path, "unknown row filter");
                break;
            }
            unsigned char *cur = row + 1;
            const unsigned char *up = y ? raw + (size_t)(y - 1) * (stride + 1) + 1 : NULL;
            for (size_t i = 0; i < stride; ++i) {
                const int a = i >= (size_t)spp ? cur[i - spp] : 0;
                const int b = up ? up[i] : 0;
                const int cc = (up && i >= (size_t)spp) ? up[i - spp] : 0;
                int v = cur[i];
                switch (ft) {
                case 0: break;
                case 1: v += a; break;
                case 2: v += b; break;
                case 3: v += (a + b) >> 1; break;
                default: v += paeth(a, b, cc); break;
                }
                cur[i] = (unsigned char)v;
            }
        }
    }
    unsigned char *out = NULL;
    if (rc == ACH_OK) {
        out = (unsigned char *)malloc((size_t)W * H * chans);
        if (!out) rc = fail(path, "out of host memory");
    }
    if (rc == ACH_OK) {
        for (int y = 0; y < H; ++y) {
            const unsigned char *cur = raw + (size_t)y * (stride + 1) + 1;
            unsigned char *o = out + (size_t)y * W * chans;
            for (int x = 0; x < W; ++x)
                for (int k = 0; k < chans; ++k) {
                    if (ctype == 3) {
                        const int idx = cur[x];
                        if (idx >= npal) {
                            rc = fail(path, "palette index out of range");
                            goto done;
                        }
                        o[(size_t)x * chans + k] = pal[idx][k];
                    } else {
                        o[(size_t)x * chans + k] = cur[(size_t)x * chans + k];
                    }
                }
        }
    }
done:
    free(raw);
    free(idat);
    if (rc != ACH_OK) {
        free(out);
        return rc;
    }
    *Wp = W;
    *Hp = H;
    *chansp = chans;
    *px = out;
    return ACH_OK;
}

/* binary PPM (P6, 3 channels) / PGM (P5, 1 channel), maxval 255 */
static int decode_pnm(const char *path, const unsigned char *buf, size_t len, int *Wp, int *Hp,
                      int *chansp, unsigned char **px)
{
    const int chans = buf[1] == '6' ? 3 : 1;
    size_t pos = 2;
    int vals[3], nv = 0;
    while (nv < 3 && pos < len) {
        const unsigned char ch = buf[pos];
        if (ch == '#') {
            while (pos < len && buf[pos] != '\n') ++pos;
        } else if (ch >= '0' && ch <= '9') {
            long v = 0;
            while (pos < len && buf[pos] >= '0' && buf[pos] <= '9' && v < 1 << 24)
                v = v * 10 + (buf[pos++] - '0');
            vals[nv++] = (int)v;
            continue;
        } else if (ch != ' ' && ch != '\t' && ch != '\n' && ch != '\r') {
            return fail(path, "bad PNM header");
        }
        ++pos;
    }
    if (nv < 3 || pos >= len) return fail(path, "bad PNM header");
    ++pos; /* the single whitespace after maxval */
    if (vals[2] != 255) return fail(path, "only maxval 255 is supported");
    if (vals[0] <= 0 || vals[1] <= 0 || vals[0] > (1 << 15) || vals[1] > (1 << 15))
        return fail(path, "image size out of range");
    const size_t n = (size_t)vals[0] * vals[1] * chans;
    if (len - pos < n) return fail(path, "truncated image data");
    unsigned char *out = (unsigned char *)malloc(n);
    if (!out) return fail(path, "out of host memory");
    memcpy(out, buf + pos, n);
    *Wp = vals[0];
    *Hp = vals[1];
    *chansp = chans;
    *px = out;
    return ACH_OK;
}

/* the file's pixels at their native size and channel count */
static int decode_file(const char *path, int *W, int *H, int *chans, unsigned char **px)
{
    size_t len = 0;
    unsigned char *buf = read_file(path, &len);
    if (!buf) return fail(path, "cannot read");
    int rc;
    if (len >= 8 && buf[0] == 137 && buf[1] == 'P' && buf[2] == 'N' && buf[3] == 'G')
        rc = decode_png(path, buf, len, W, H, chans, px);
    else if (len >= 3 && buf[0] == 'P' && (buf[1] == '5' || buf[1] == '6'))
        rc = decode_pnm(path, buf, len, W, H, chans, px);
    else if (len >= 3 && buf[0] == 0xff && buf[1] == 0xd8 && buf[2] == 0xff) {
        const char *why = NULL;
        rc = an_jpeg_decode(buf, len, W, H, chans, px, &why) ? fail(path, why) : ACH_OK;
    } else
        rc = fail(path, "unsupported format (PNG, JPEG, binary PPM / PGM)");
    free(buf);
    return rc;
}

/* interleaved 8-bit samples -> planar floats / 255 (NImage.reload's loop) */
static void to_planes(const unsigned char *px, int W, int H, int c, float *dst)
{
    const size_t plane = (size_t)W * H;
    for (size_t p = 0; p < plane; ++p)
        for (int k = 0; k < c; ++k) dst[k * plane + p] = (float)px[p * c + k] / 255.0f;
}

int an_image_load(const char *path, int w, int h, int c, float *dst)
{
    if (!path || !dst || w <= 0 || h <= 0 || c <= 0) return ACH_EINVAL;
    int W, H, chans;
    unsigned char *px = NULL;
    int rc = decode_file(path, &W, &H, &chans, &px);
    if (rc) return rc;
    /* NImage.reload: the file must have the network's size and channels */
    if (W != w || H != h || chans != c)
        rc = fail(path, "image size or channel count differs from the network input");
    else
        to_planes(px, W, H, c, dst);
    free(px);
    return rc;
}

/* The channel conversion of stb_image's loader when a channel count is
 * requested (the reference's NImage.createImage asks for 3): grey is
 * replicated, alpha dropped or set opaque, and RGB turns grey as
 * (77 r + 150 g + 29 b) >> 8.                                               */
static unsigned char luma(const unsigned char *p)
{
    return (unsigned char)((p[0] * 77 + p[1] * 150 + p[2] * 29) >> 8);
}

static void convert_channels(const unsigned char *in, int from, unsigned char *out, int to,
                             size_t npix)
{
    for (size_t i = 0; i < npix; ++i) {
        const unsigned char *s = in + i * from;
        unsigned char *d = out + i * to;
        unsigned char g, a = 255, rgb[3];
        switch (from) {
        case 1: g = s[0]; rgb[0] = rgb[1] = rgb[2] = g; break;
        case 2: g = s[0]; a = s[1]; rgb[0] = rgb[1] = rgb[2] = g; break;
        case 3: rgb[0] = s[0]; rgb[1] = s[1]; rgb[2] = s[2]; g = luma(s); break;
        default: rgb[0] = s[0]; rgb[1] = s[1]; rgb[2] = s[2]; a = s[3]; g = luma(s); break;
        }
        switch (to) {
        case 1: d[0] = g; break;
        case 2: d[0] = g; d[1] = a; break;
        case 3: d[0] = rgb[0]; d[1] = rgb[1]; d[2] = rgb[2]; break;
        default: d[0] = rgb[0]; d[1] = rgb[1]; d[2] = rgb[2]; d[3] = a; break;
        }
    }
}

int an_image_read(const char *path, int c, int *w, int *h, float **dst)
{
    if (!path || !w || !h || !dst || c < 1 || c > 4) return ACH_EINVAL;
    int W, H, chans;
    unsigned char *px = NULL;
    int rc = decode_file(path, &W, &H, &chans, &px);
    if (rc) return rc;
    unsigned char *cv = px;
    if (chans != c) {
        cv = (unsigned char *)malloc((size_t)W * H * c);
        if (!cv) {
            free(px);
            return fail(path, "out of host memory");
        }
        convert_channels(px, chans, cv, c, (size_t)W * H);
    }
    float *out = (float *)malloc(sizeof(float) * (size_t)W * H * c);
    if (!out) rc = fail(path, "out of host memory");
    else to_planes(cv, W, H, c, out);
    if (cv != px) free(cv);
    free(px);
    if (rc) return rc;
    *w = W;
    *h = H;
    *dst = out;
    return ACH_OK;
}

void an_image_free(float *im) { free(im); }

/* NImage.resizeMin (NImage.c:1037-1051): the size whose smaller side is min,
 * the other scaled in integer arithmetic                                     */
void an_image_resize_min_size(int W, int H, int min, int *w, int *h)
{
    if (W < H) {
        *h = (H * min) / W;
        *w = min;
    } else {
        *w = (W * min) / H;
        *h = min;
    }
}

/* NImage.crop (NImage.c:439-458): the w x h window at (dx, dy), coordinates
 * clamped to the image                                                      */
void an_image_crop(const float *src, int W, int H, int c, int dx, int dy, int w, int h,
                   float *dst)
{
    for (int k = 0; k < c; ++k)
        for (int j = 0; j < h; ++j) {
            int r = j + dy;
            r = r < 0 ? 0 : (r > H - 1 ? H - 1 : r);
            for (int i = 0; i < w; ++i) {
                int cc = i + dx;
                cc = cc < 0 ? 0 : (cc > W - 1 ? W - 1 : cc);
                dst[(size_t)k * w * h + (size_t)j * w + i] =
                    src[(size_t)k * W * H + (size_t)r * W + cc];
            }
        }
}

/* ---- labels from paths (ImageData.fillTruthSmooth, ImageData.c:80-104) ----- */
int an_label_from_path(const char *path, const char *const *labels, int nlabels)
{
    if (!path || !labels || nlabels <= 0) return -1;
    int found = -1, count = 0;
    for (int i = 0; i < nlabels; ++i)
        if (labels[i] && strstr(path, labels[i])) {
            found = i;
            ++count;
        }
    return count == 1 ? found : -1;
}

/* ---- augmentation -------------------------------------------------------- */
void an_augment_defaults(an_augment *a, int net_w)
{
    /* parseNetOption (NetworkFactory.c:727-762) */
    a->min_crop = net_w;
    a->max_crop = 2 * net_w;
    a->angle = 0.f;
    a->aspect = 1.f;
    a->hue = 0.f;
    a->saturation = 1.f;
    a->exposure = 1.f;
    a->flip = 1;
}

/* the reference's generators over the counter-based stream */
#define AUG_RAND_MAX 2147483647u
enum {
    SALT_ASPECT = 4, SALT_ASPECT_INV, SALT_CROP, SALT_ANGLE, SALT_DX, SALT_DY, SALT_FLIP,
    SALT_HUE, SALT_SAT, SALT_SAT_INV, SALT_EXP, SALT_EXP_INV
};

typedef struct {
    uint64_t seed, batch_no;
    int image;
} aug_rng;

static uint32_t rnd(const aug_rng *r, int salt) /* rand(): [0, 2^31 - 1] */
{
    return (uint32_t)(an_feeder_sample(r->seed, r->batch_no, r->image, salt) >> 33);
}

static float rand_uniform(const aug_rng *r, int salt, float min, float max) /* DnnUtils.c:196-209 */
{
    if (max < min) {
        const float s = min;
        min = max;
        max = s;
    }
    return ((float)rnd(r, salt) / AUG_RAND_MAX * (max - min)) + min;
}

static float rand_uniform_strong(const aug_rng *r, int salt, float min, float max)
{
    if (max < min) { /* DnnUtils.h:94-101, randomFloat DnnUtils.h:84-92 */
        const float s = min;
        min = max;
        max = s;
    }
    return ((float)rnd(r, salt) / (float)AUG_RAND_MAX) * (max - min) + min;
}

static float rand_scale(const aug_rng *r, int salt, int salt_inv, float s) /* DnnUtils.c:188-193 */
{
    const float scale = rand_uniform_strong(r, salt, 1, s);
    if (rnd(r, salt_inv) % 2) return scale;
    return 1. / scale;
}

static int rand_int(const aug_rng *r, int salt, int min, int max) /* DnnUtils.c:224-232 */
{
    if (max < min) {
        const int s = min;
        min = max;
        max = s;
    }
    return (int)(rnd(r, salt) % (uint32_t)(max - min + 1)) + min;
}

/* getPixelExtend + bilinearInterpolate (NImage.c:138-158) */
static float pixel_ext(const float *im, int W, int H, int x, int y, int k)
{
    if (x < 0 || x >= W || y < 0 || y >= H) return 0;
    return im[(size_t)k * W * H + (size_t)y * W + x];
}

static float bilinear(const float *im, int W, int H, float x, float y, int k)
{
    const int ix = (int)floorf(x), iy = (int)floorf(y);
    const float dx = x - ix, dy = y - iy;
    return (1 - dy) * (1 - dx) * pixel_ext(im, W, H, ix, iy, k) +
           dy * (1 - dx) * pixel_ext(im, W, H, ix, iy + 1, k) +
           (1 - dy) * dx * pixel_ext(im, W, H, ix + 1, iy, k) +
           dy * dx * pixel_ext(im, W, H, ix + 1, iy + 1, k);
}

void an_image_rotate_crop(const float *src, int W, int H, int c, float rad, float s, int w, int h,
                          float dx, float dy, float aspect, float *dst)
{
    /* NImage.rotateCrop (NImage.c:551-572) */
    const float cx = W / 2.0, cy = H / 2.0;
    const float cr = cos(rad), sr = sin(rad);
    const float dx1 = dx / s * aspect, dy1 = dy / s;
    for (int k = 0; k < c; ++k)
        for (int y = 0; y < h; ++y)
            for (int x = 0; x < w; ++x) {
                /* the reference's expressions, evaluated in double */
                const float rx = cr * ((x - w / 2.) / s * aspect + dx1) - sr * ((y - h / 2.) / s + dy1) + cx;
                const float ry = sr * ((x - w / 2.) / s * aspect + dx1) + cr * ((y - h / 2.) / s + dy1) + cy;
                dst[(size_t)k * w * h + (size_t)y * w + x] = bilinear(src, W, H, rx, ry, k);
            }
}

void an_image_flip(float *im, int w, int h, int c)
{
    for (int k = 0; k < c; ++k) /* NImage.flip (NImage.c:355-370) */
        for (int i = 0; i < h; ++i)
            for (int j = 0; j < w / 2; ++j) {
                float *row = im + (size_t)k * w * h + (size_t)i * w;
                const float t = row[w - j - 1];
                row[w - j - 1] = row[j];
                row[j] = t;
            }
}

static float max3(float a, float b, float c) { return (a > b) ? ((a > c) ? a : c) : ((b > c) ? b : c); }
static float min3(float a, float b, float c) { return (a < b) ? ((a < c) ? a : c) : ((b < c) ? b : c); }

void an_image_distort(float *im, int w, int h, float hue, float sat, float val)
{
    /* NImage.distort (NImage.c:323-338): RGB -> HSV (:201-243), s *= sat,
     * v *= val, h += hue wrapped into [0, 1], HSV -> RGB (:245-292), clamp */
    const size_t plane = (size_t)w * h;
    float *R = im, *G = im + plane, *B = im + 2 * plane;
    for (size_t p = 0; p < plane; ++p) {
        const float r = R[p], g = G[p], b = B[p];
        const float mx = max3(r, g, b), mn = min3(r, g, b), delta = mx - mn;
        float hh, s, v = mx;
        if (mx == 0) {
            s = 0;
            hh = 0;
        } else {
            s = delta / mx;
            if (r == mx) hh = (g - b) / delta;
            else if (g == mx) hh = 2 + (b - r) / delta;
            else hh = 4 + (r - g) / delta;
            if (hh < 0) hh += 6;
            hh = hh / 6.;
        }
        s = s * sat;
        v = v * val;
        hh = hh + hue;
        if (hh > 1) hh -= 1;
        if (hh < 0) hh += 1;
        /* hsvToRgb */
        float ro, go, bo;
        hh = 6 * hh;
        if (s == 0) {
            ro = go = bo = v;
        } else {
            const int index = (int)floor(hh);
            const float f = hh - index, pp = v * (1 - s), q = v * (1 - s * f),
                        t = v * (1 - s * (1 - f));
            if (index == 0) { ro = v; go = t; bo = pp; }
            else if (index == 1) { ro = q; go = v; bo = pp; }
            else if (index == 2) { ro = pp; go = v; bo = t; }
            else if (index == 3) { ro = pp; go = q; bo = v; }
            else if (index == 4) { ro = t; go = pp; bo = v; }
            else { ro = v; go = pp; bo = q; }
        }
        R[p] = ro < 0 ? 0 : (ro > 1 ? 1 : ro);
        G[p] = go < 0 ? 0 : (go > 1 ? 1 : go);
        B[p] = bo < 0 ? 0 : (bo > 1 ? 1 : bo);
    }
}

int an_image_resize(const float *src, int W, int H, int c, int w, int h, float *dst)
{
    /* NImage.resizeImage (NImage.c:474-530): rows first, then columns */
    if (!src || !dst || W <= 0 || H <= 0 || c <= 0 || w <= 0 || h <= 0) return ACH_EINVAL;
    if (W == w && H == h) {
        memcpy(dst, src, sizeof(float) * (size_t)w * h * c);
        return ACH_OK;
    }
    float *part = (float *)malloc(sizeof(float) * (size_t)w * H * c);
    if (!part) return ACH_EINVAL;
    /* a one-pixel output side samples source row / column 0 (the
     * reference's (H-1)/(h-1) would divide by zero there) */
    const float w_scale = w > 1 ? (float)(W - 1) / (w - 1) : 0.f;
    const float h_scale = h > 1 ? (float)(H - 1) / (h - 1) : 0.f;
    for (int k = 0; k < c; ++k)
        for (int r = 0; r < H; ++r)
            for (int x = 0; x < w; ++x) {
                const float *row = src + (size_t)k * W * H + (size_t)r * W;
                float val;
                if (x == w - 1 || W == 1) {
                    val = row[W - 1];
                } else {
                    const float sx = x * w_scale;
                    const int ix = (int)sx;
                    const float dx = sx - ix;
                    val = (1 - dx) * row[ix] + dx * row[ix + 1];
                }
                part[(size_t)k * w * H + (size_t)r * w + x] = val;
            }
    for (int k = 0; k < c; ++k)
        for (int r = 0; r < h; ++r) {
            const float sy = r * h_scale;
            const int iy = (int)sy;
            const float dy = sy - iy;
            float *out = dst + (size_t)k * w * h + (size_t)r * w;
            const float *p0 = part + (size_t)k * w * H + (size_t)iy * w;
            for (int x = 0; x < w; ++x) out[x] = (1 - dy) * p0[x];
            if (r == h - 1 || H == 1) continue;
            for (int x = 0; x < w; ++x) out[x] += dy * p0[x + w];
        }
    free(part);
    return ACH_OK;
}

int an_augment_image(const float *src, int w, int h, int c, const an_augment *a, uint64_t seed,
                     uint64_t batch_no, int image, float *dst)
{
    if (!src || !dst || !a || w <= 0 || h <= 0 || c <= 0 || a->min_crop <= 0 ||
        a->max_crop <= 0)
        return ACH_EINVAL;
    const aug_rng r = {seed, batch_no, image};
    const int size = w > h ? w : h;
    /* NImage.randomAugment (NImage.c:1016-1034) */
    const float aspect = rand_scale(&r, SALT_ASPECT, SALT_ASPECT_INV, a->aspect);
    const int crop = rand_int(&r, SALT_CROP, a->min_crop, a->max_crop);
    const int mn = (h < w * aspect) ? h : (int)(w * aspect);
    const float scale = (float)crop / mn;
    const float rad = rand_uniform(&r, SALT_ANGLE, -a->angle, a->angle) * 2.0 * M_PI / 360.;
    float dx = (w * scale / aspect - size) / 2., dy = (h * scale - size) / 2.;
    if (dx < 0) dx = 0;
    if (dy < 0) dy = 0;
    dx = rand_uniform(&r, SALT_DX, -dx, dx);
    dy = rand_uniform(&r, SALT_DY, -dy, dy);
    float *tmp = (float *)malloc(sizeof(float) * (size_t)size * size * c);
    if (!tmp) return ACH_EINVAL;
    an_image_rotate_crop(src, w, h, c, rad, scale, size, size, dx, dy, aspect, tmp);
    /* ImageData.loadImageAugmentPaths (ImageData.c:63-70): flip, distort, resize */
    if (a->flip && rnd(&r, SALT_FLIP) % 2) an_image_flip(tmp, size, size, c);
    if (c == 3) { /* rgbToHsv asserts 3 channels (NImage.c:202) */
        const float dhue = rand_uniform_strong(&r, SALT_HUE, -a->hue, a->hue);
        const float dsat = rand_scale(&r, SALT_SAT, SALT_SAT_INV, a->saturation);
        const float dexp = rand_scale(&r, SALT_EXP, SALT_EXP_INV, a->exposure);
        an_image_distort(tmp, size, size, dhue, dsat, dexp);
    }
    const int rc = an_image_resize(tmp, size, size, c, w, h, dst);
    free(tmp);
    return rc;
}
