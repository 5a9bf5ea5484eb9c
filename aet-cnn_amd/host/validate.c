/*
 * validate.c -- top-1 / top-k accuracy over a list of labelled images, the
 * reference's Classifier.validateSingle (Classifier.c:359-464; paths under
 * /root/reference/src/com/ai/dnn/):
 *
 *   for every path of the list:  class = the first label that is a
 *   substring of the path (-1: none, counted as a miss);  the image loaded
 *   at its own size with the network's channel count (NImage.createImage,
 *   NImage.c:587-623), resized so its smaller side is the network width
 *   (NImage.resizeMin, NImage.c:1037-1051), the network's w x h window cut
 *   from its centre (NImage.crop, NImage.c:439-458), predicted, and the k
 *   best classes taken (DnnUtils.topK, DnnUtils.c:463-477).
 *
 * The reference predicts one image at a time on a batch-1 network; here the
 * images fill the network's batch (inference is per image: batch-norm on the
 * rolling statistics, no dropout), a last partial batch padded with zero
 * images whose outputs are ignored.  Its class-tree (hierarchy) branch is
 * not carried over: the tree softmax is not built.
 */
#include "aetcnn_net.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define AN_CHECK(expr)                 \
    do {                               \
        int rc_ = (expr);              \
        if (rc_ != ACH_OK) return rc_; \
    } while (0)

static void free_paths(char **paths, int n)
{
    for (int i = 0; i < n; ++i) free(paths[i]);
    free(paths);
}

/* the non-empty lines of a list file (trailing spaces and CR/LF removed) */
static char **read_paths(const char *list_file, int *count)
{
    FILE *fp = fopen(list_file, "r");
    if (!fp) {
        fprintf(stderr, "an_validate_paths: cannot open %s\n", list_file);
        return NULL;
    }
    char line[4096];
    char **paths = NULL;
    int n = 0, cap = 0, ok = 1;
    while (ok && fgets(line, sizeof(line), fp)) {
        size_t len = strlen(line);
        while (len && (line[len - 1] == '\n' || line[len - 1] == '\r' || line[len - 1] == ' '))
            line[--len] = 0;
        if (!len) continue;
        if (n == cap) {
            cap = cap ? 2 * cap : 256;
            char **np = (char **)realloc(paths, (size_t)cap * sizeof(char *));
            if (!np) {
                ok = 0;
                break;
            }
            paths = np;
        }
        paths[n] = strdup(line);
        if (!paths[n]) ok = 0;
        else ++n;
    }
    fclose(fp);
    if (!ok) {
        free_paths(paths, n);
        return NULL;
    }
    *count = n;
    return paths;
}

/* one image as the network's input: native size, resize-min, centre crop */
int an_validation_image(const char *path, int w, int h, int c, float *dst)
{
    if (!path || !dst || w <= 0 || h <= 0 || c <= 0 || c > 4) return ACH_EINVAL;
    int W = 0, H = 0;
    float *im = NULL;
    AN_CHECK(an_image_read(path, c, &W, &H, &im));
    int rw, rh;
    an_image_resize_min_size(W, H, w, &rw, &rh);
    float *rs = (float *)malloc(sizeof(float) * (size_t)rw * rh * c);
    if (!rs) {
        an_image_free(im);
        return ACH_EINVAL;
    }
    const int rc = an_image_resize(im, W, H, c, rw, rh, rs);
    if (rc == ACH_OK) an_image_crop(rs, rw, rh, c, (rw - w) / 2, (rh - h) / 2, w, h, dst);
    free(rs);
    an_image_free(im);
    return rc;
}

int an_validate_paths(an_network *net, const char *list_file, const char *const *labels,
                      int nlabels, int topk, an_validation *result)
{
    if (!net || !list_file || !labels || nlabels <= 0 || topk <= 0 || !result)
        return ACH_EINVAL;
    int shape[8];
    AN_CHECK(an_layer_shape(net, 0, shape));
    const int c = shape[4], h = shape[5], w = shape[6];
    const int B = an_batch(net), classes = an_classes(net);
    if (B <= 0 || classes <= 0) return ACH_EINVAL;
    if (topk > classes) topk = classes;
    int npaths = 0;
    char **paths = read_paths(list_file, &npaths);
    if (!paths) return ACH_EINVAL;
    const size_t img = (size_t)w * h * c;
    float *in = (float *)calloc((size_t)B * img, sizeof(float));
    float *out = (float *)malloc(sizeof(float) * (size_t)B * classes);
    int *cls = (int *)malloc(sizeof(int) * (size_t)B);
    int *idx = (int *)malloc(sizeof(int) * (size_t)topk);
    int rc = (in && out && cls && idx) ? ACH_OK : ACH_EINVAL;
    long hit1 = 0, hitk = 0, unlabeled = 0;
    for (int start = 0; rc == ACH_OK && start < npaths; start += B) {
        const int nb = npaths - start < B ? npaths - start : B;
        for (int i = 0; rc == ACH_OK && i < nb; ++i) {
            const char *path = paths[start + i];
            cls[i] = -1;
            for (int j = 0; j < nlabels; ++j)
                if (labels[j] && strstr(path, labels[j])) {
                    cls[i] = j;
                    break;
                }
            if (cls[i] < 0) ++unlabeled;
            rc = an_validation_image(path, w, h, c, in + (size_t)i * img);
        }
        if (rc) break;
        if (nb < B) memset(in + (size_t)nb * img, 0, sizeof(float) * (size_t)(B - nb) * img);
        rc = an_predict(net, in, out);
        for (int i = 0; rc == ACH_OK && i < nb; ++i) {
            an_top_k(out + (size_t)i * classes, classes, topk, idx);
            if (idx[0] == cls[i]) ++hit1;
            for (int j = 0; j < topk; ++j)
                if (idx[j] == cls[i]) ++hitk;
        }
    }
    free(in);
    free(out);
    free(cls);
    free(idx);
    free_paths(paths, npaths);
    if (rc) return rc;
    result->images = npaths;
    result->unlabeled = (int)unlabeled;
    result->topk = topk;
    /* float counts divided as the reference's avg_acc / avg_topk */
    result->top1_accuracy = npaths ? (float)hit1 / (float)npaths : 0.f;
    result->topk_accuracy = npaths ? (float)hitk / (float)npaths : 0.f;
    return ACH_OK;
}
