/* Input pipeline: worker threads decode batches into pinned host slots, the
 * host-to-device copy of batch k+1 runs on its own stream while the GPU
 * trains on batch k.
 *
 * Reference behaviour replaced (paths under /root/reference/src/com/ai/dnn/):
 *   ImageData (ImageData.c:20-224): a thread pool (DstbCompute.c:60-216)
 *   fills one half of a two-batch host buffer while training reads the other
 *   (loadData / wait / getNextBatch); each image is drawn at random from the
 *   training set (getRandomPaths, ImageData.c:37-51), optionally flipped
 *   (loadImageAugmentPaths, :54-71), and its one-hot truth is written with
 *   label smoothing (fillTruthSmooth, :77-103).  Classifier.train
 *   (Classifier.c:216-243) sets it up with 12 threads.
 *
 * Sources: a list of image files with labels from substrings of the path,
 * as the reference reads its training set (getPaths, fillTruthSmooth; PNG /
 * PPM / PGM decoded by image.c), the CIFAR-10 binary batches (1 label byte
 * + 3x32x32 planar RGB bytes per record; the same images and labels), or
 * synthetic pixels.  Every image then takes the reference's augmentation
 * (loadImageAugmentPaths: random scale / aspect / rotation crop, flip,
 * hue / saturation / exposure distortion; an_augment_image in image.c)
 * when the feeder has an an_augment.  The image index and every random draw
 * of image i of batch k come from a counter-based hash of (seed, k, i)
 * instead of the shared rand() stream, so the batches do not depend on
 * thread scheduling.                                                        */
#include "aetcnn_net.h"

#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define CIFAR_REC 3073
#define CIFAR_SIDE 32

enum { SRC_SYNTHETIC = 0, SRC_CIFAR = 1, SRC_PATHS = 2 };
enum { SLOT_IDLE = 0, SLOT_FILLING = 1, SLOT_READY = 2 };

struct an_feeder {
    an_network *net;
    int batch, inputs, classes, c, h, w;
    int kind;
    unsigned char *records; /* CIFAR records, nrecords x 3073 bytes */
    size_t nrecords;
    char **paths;           /* image files and their labels (SRC_PATHS) */
    int *path_label;
    size_t npaths;
    uint64_t seed;
    int augment;
    an_augment aug;
    float smooth;
    int load_error;         /* a worker could not decode an image */
    float *host_in[2], *host_truth[2]; /* pinned */
    float *dev_in[2], *dev_truth[2];
    void *copied[2];
    ach_stream_t copy_stream;
    uint64_t slot_batch[2];
    int state[2];
    int next_img[2], done_img[2];
    uint64_t served;
    pthread_t *threads;
    int nthreads;
    pthread_mutex_t mu;
    pthread_cond_t cv_work, cv_ready;
    int stop;
};

/* SplitMix64 finaliser (Steele, Lea, Flood 2014) */
static uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static uint64_t draw(uint64_t seed, uint64_t batch_no, uint64_t i, uint64_t salt)
{
    return mix64(seed + 0x9E3779B97F4A7C15ull * (batch_no + 1) + mix64(i * 4 + salt));
}

uint64_t an_feeder_sample(uint64_t seed, uint64_t batch_no, int image, int what)
{
    return draw(seed, batch_no, (uint64_t)image, (uint64_t)what);
}

static void fill_truth(float *truth, int classes, int label, float eps)
{
    for (int k = 0; k < classes; ++k)
        truth[k] = (k == label) ? 1.f - eps : (classes > 1 ? eps / (classes - 1) : 0.f);
}

/* image i of batch bn into slot s: the source image (into `tmp` when it is
 * augmented afterwards, else straight into the slot), then the augmentation;
 * returns ACH_OK or the decoder's error */
static int fill_image(an_feeder *f, int s, uint64_t bn, int i, float *tmp)
{
    float *img = f->host_in[s] + (size_t)i * f->inputs;
    float *truth = f->host_truth[s] + (size_t)i * f->classes;
    float *src = f->augment ? tmp : img;
    int label;
    if (f->kind == SRC_CIFAR) {
        const size_t idx = (size_t)(draw(f->seed, bn, (uint64_t)i, 0) % f->nrecords);
        const unsigned char *rec = f->records + idx * CIFAR_REC;
        for (int j = 0; j < 3 * CIFAR_SIDE * CIFAR_SIDE; ++j) src[j] = rec[1 + j] / 255.f;
        label = rec[0];
    } else if (f->kind == SRC_PATHS) {
        const size_t idx = (size_t)(draw(f->seed, bn, (uint64_t)i, 0) % f->npaths);
        const int rc = an_image_load(f->paths[idx], f->w, f->h, f->c, src);
        if (rc) return rc;
        label = f->path_label[idx];
    } else {
        for (int j = 0; j < f->inputs; ++j)
            src[j] = (float)(draw(f->seed, bn, (uint64_t)i * (uint64_t)f->inputs + j, 2) >> 40) *
                     (1.0f / 16777216.0f);
        label = (int)(draw(f->seed, bn, (uint64_t)i, 3) % f->classes);
    }
    fill_truth(truth, f->classes, label, f->smooth);
    if (!f->augment) return ACH_OK;
    return an_augment_image(src, f->w, f->h, f->c, &f->aug, f->seed, bn, i, img);
}

static void *worker(void *arg)
{
    an_feeder *f = (an_feeder *)arg;
    const int chunk = f->batch / (2 * f->nthreads) > 0 ? f->batch / (2 * f->nthreads) : 1;
    float *tmp = (float *)malloc(sizeof(float) * (size_t)f->inputs);
    pthread_mutex_lock(&f->mu);
    for (;;) {
        int s = -1;
        while (!f->stop) {
            for (int k = 0; k < 2; ++k)
                if (f->state[k] == SLOT_FILLING && f->next_img[k] < f->batch) {
                    s = k;
                    break;
                }
            if (s >= 0) break;
            pthread_cond_wait(&f->cv_work, &f->mu);
        }
        if (f->stop) break;
        const int lo = f->next_img[s];
        const int hi = lo + chunk < f->batch ? lo + chunk : f->batch;
        f->next_img[s] = hi;
        const uint64_t bn = f->slot_batch[s];
        pthread_mutex_unlock(&f->mu);
        int err = tmp ? ACH_OK : ACH_EINVAL;
        for (int i = lo; i < hi && !err; ++i) err = fill_image(f, s, bn, i, tmp);
        pthread_mutex_lock(&f->mu);
        if (err) { /* wake an_feeder_next, which reports the failure */
            f->load_error = 1;
            pthread_cond_broadcast(&f->cv_ready);
        }
        f->done_img[s] += hi - lo;
        if (f->done_img[s] == f->batch) {
            f->state[s] = SLOT_READY;
            pthread_cond_broadcast(&f->cv_ready);
        }
    }
    pthread_mutex_unlock(&f->mu);
    free(tmp);
    return NULL;
}

/* caller holds mu */
static void start_fill(an_feeder *f, int s, uint64_t bn)
{
    f->slot_batch[s] = bn;
    f->next_img[s] = 0;
    f->done_img[s] = 0;
    f->state[s] = SLOT_FILLING;
    pthread_cond_broadcast(&f->cv_work);
}

void an_feeder_free(an_feeder *f)
{
    if (!f) return;
    if (f->threads) {
        pthread_mutex_lock(&f->mu);
        f->stop = 1;
        pthread_cond_broadcast(&f->cv_work);
        pthread_mutex_unlock(&f->mu);
        for (int t = 0; t < f->nthreads; ++t) pthread_join(f->threads[t], NULL);
        free(f->threads);
    }
    if (f->copy_stream) ach_stream_sync(f->copy_stream);
    for (int s = 0; s < 2; ++s) {
        ach_host_free(f->host_in[s]);
        ach_host_free(f->host_truth[s]);
        ach_free(f->dev_in[s]);
        ach_free(f->dev_truth[s]);
        if (f->copied[s]) ach_event_destroy(f->copied[s]);
    }
    if (f->copy_stream) ach_stream_destroy(f->copy_stream);
    pthread_mutex_destroy(&f->mu);
    pthread_cond_destroy(&f->cv_work);
    pthread_cond_destroy(&f->cv_ready);
    free(f->records);
    for (size_t k = 0; k < f->npaths; ++k) free(f->paths[k]);
    free(f->paths);
    free(f->path_label);
    free(f);
}

static an_feeder *feeder_new(an_network *net, int threads, uint64_t seed, const an_augment *aug,
                             float label_smooth_eps)
{
    int shape[8];
    if (!net || threads <= 0 || threads > 256 || !(label_smooth_eps >= 0.f) ||
        label_smooth_eps >= 1.f || an_layer_shape(net, 0, shape) != ACH_OK || an_batch(net) <= 0)
        return NULL;
    an_feeder *f = (an_feeder *)calloc(1, sizeof(an_feeder));
    if (!f) return NULL;
    f->net = net;
    f->batch = an_batch(net);
    f->c = shape[4];
    f->h = shape[5];
    f->w = shape[6];
    f->inputs = f->c * f->h * f->w;
    f->classes = an_classes(net);
    f->seed = seed;
    f->augment = aug != NULL;
    if (aug) f->aug = *aug;
    f->smooth = label_smooth_eps;
    f->nthreads = threads;
    pthread_mutex_init(&f->mu, NULL);
    pthread_cond_init(&f->cv_work, NULL);
    pthread_cond_init(&f->cv_ready, NULL);
    if (aug && (aug->min_crop <= 0 || aug->max_crop <= 0)) {
        an_feeder_free(f);
        return NULL;
    }
    return f;
}

static an_feeder *feeder_start(an_feeder *f)
{
    const size_t in_bytes = sizeof(float) * (size_t)f->batch * f->inputs;
    const size_t tr_bytes = sizeof(float) * (size_t)f->batch * f->classes;
    if (f->classes <= 0 || ach_stream_create(&f->copy_stream) != ACH_OK) goto fail;
    for (int s = 0; s < 2; ++s) {
        if (ach_host_alloc((void **)&f->host_in[s], in_bytes) != ACH_OK ||
            ach_host_alloc((void **)&f->host_truth[s], tr_bytes) != ACH_OK ||
            ach_malloc((void **)&f->dev_in[s], in_bytes) != ACH_OK ||
            ach_malloc((void **)&f->dev_truth[s], tr_bytes) != ACH_OK ||
            ach_event_create(&f->copied[s]) != ACH_OK)
            goto fail;
    }
    f->threads = (pthread_t *)calloc((size_t)f->nthreads, sizeof(pthread_t));
    if (!f->threads) goto fail;
    for (int t = 0; t < f->nthreads; ++t)
        if (pthread_create(&f->threads[t], NULL, worker, f) != 0) {
            f->nthreads = t;
            goto fail;
        }
    pthread_mutex_lock(&f->mu);
    start_fill(f, 0, 0);
    start_fill(f, 1, 1);
    pthread_mutex_unlock(&f->mu);
    return f;
fail:
    an_feeder_free(f);
    return NULL;
}

an_feeder *an_feeder_create_cifar(an_network *net, const char *const *files, int nfiles,
                                  int threads, uint64_t seed, const an_augment *aug,
                                  float label_smooth_eps)
{
    an_feeder *f = feeder_new(net, threads, seed, aug, label_smooth_eps);
    if (!f) return NULL;
    f->kind = SRC_CIFAR;
    if (!files || nfiles <= 0 || f->c != 3 || f->h != CIFAR_SIDE || f->w != CIFAR_SIDE ||
        f->classes < 10) {
        fprintf(stderr, "an_feeder_create_cifar: network input must be 3x32x32 with >= 10 "
                        "classes\n");
        an_feeder_free(f);
        return NULL;
    }
    size_t cap = 0;
    for (int k = 0; k < nfiles; ++k) {
        FILE *fp = fopen(files[k], "rb");
        if (!fp) {
            fprintf(stderr, "an_feeder_create_cifar: cannot open %s\n", files[k]);
            an_feeder_free(f);
            return NULL;
        }
        unsigned char rec[CIFAR_REC];
        while (fread(rec, 1, CIFAR_REC, fp) == CIFAR_REC) {
            if (rec[0] >= f->classes) continue;
            if (f->nrecords == cap) {
                cap = cap ? 2 * cap : 16384;
                unsigned char *nr = (unsigned char *)realloc(f->records, cap * CIFAR_REC);
                if (!nr) {
                    fclose(fp);
                    an_feeder_free(f);
                    return NULL;
                }
                f->records = nr;
            }
            memcpy(f->records + f->nrecords * CIFAR_REC, rec, CIFAR_REC);
            ++f->nrecords;
        }
        fclose(fp);
    }
    if (f->nrecords == 0) {
        fprintf(stderr, "an_feeder_create_cifar: no records\n");
        an_feeder_free(f);
        return NULL;
    }
    return feeder_start(f);
}

an_feeder *an_feeder_create_synthetic(an_network *net, int threads, uint64_t seed,
                                      const an_augment *aug)
{
    an_feeder *f = feeder_new(net, threads, seed, aug, 0.f);
    if (!f) return NULL;
    f->kind = SRC_SYNTHETIC;
    return feeder_start(f);
}

/* The reference's training list (Classifier.c:79-108: one image path per
 * line) with labels from path substrings (fillTruthSmooth: exactly one of
 * the labels must occur in each path; checked here for the whole list). */
an_feeder *an_feeder_create_paths(an_network *net, const char *list_file,
                                  const char *const *labels, int nlabels, int threads,
                                  uint64_t seed, const an_augment *aug, float label_smooth_eps)
{
    an_feeder *f = feeder_new(net, threads, seed, aug, label_smooth_eps);
    if (!f) return NULL;
    f->kind = SRC_PATHS;
    if (!list_file || !labels || nlabels != f->classes) {
        fprintf(stderr, "an_feeder_create_paths: need a list file and one label per class "
                        "(%d)\n", f->classes);
        an_feeder_free(f);
        return NULL;
    }
    FILE *fp = fopen(list_file, "r");
    if (!fp) {
        fprintf(stderr, "an_feeder_create_paths: cannot open %s\n", list_file);
        an_feeder_free(f);
        return NULL;
    }
    char line[4096];
    size_t cap = 0;
    int ok = 1;
    while (ok && fgets(line, sizeof(line), fp)) {
        size_t n = strlen(line);
        while (n && (line[n - 1] == '\n' || line[n - 1] == '\r' || line[n - 1] == ' '))
            line[--n] = 0;
        if (!n) continue;
        const int lab = an_label_from_path(line, labels, nlabels);
        if (lab < 0) {
            fprintf(stderr, "an_feeder_create_paths: %s: too many or too few labels\n", line);
            ok = 0;
            break;
        }
        if (f->npaths == cap) {
            cap = cap ? 2 * cap : 1024;
            char **np = (char **)realloc(f->paths, cap * sizeof(char *));
            int *nl = np ? (int *)realloc(f->path_label, cap * sizeof(int)) : NULL;
            if (np) f->paths = np;
            if (nl) f->path_label = nl;
            if (!np || !nl) {
                ok = 0;
                break;
            }
        }
        f->paths[f->npaths] = strdup(line);
        f->path_label[f->npaths] = lab;
        if (!f->paths[f->npaths]) {
            ok = 0;
            break;
        }
        ++f->npaths;
    }
    fclose(fp);
    if (!ok || f->npaths == 0) {
        if (ok) fprintf(stderr, "an_feeder_create_paths: %s lists no images\n", list_file);
        an_feeder_free(f);
        return NULL;
    }
    return feeder_start(f);
}

/* Makes batch `served` the network's input: waits for its slot, copies it
 * host -> device on the feeder's stream, orders the network stream after
 * that copy and moves it into the network's input / truth there.  Once the
 * copy has left the pinned slot, the slot is refilled with batch served+2. */
int an_feeder_next(an_feeder *f)
{
    if (!f) return ACH_EINVAL;
    const int s = (int)(f->served & 1);
    pthread_mutex_lock(&f->mu);
    while (f->state[s] != SLOT_READY && !f->load_error) pthread_cond_wait(&f->cv_ready, &f->mu);
    const int bad = f->load_error;
    pthread_mutex_unlock(&f->mu);
    if (bad) return ACH_EINVAL; /* the reference aborts on an unreadable image */
    const size_t in_bytes = sizeof(float) * (size_t)f->batch * f->inputs;
    const size_t tr_bytes = sizeof(float) * (size_t)f->batch * f->classes;
    ach_stream_t ns = an_stream(f->net);
    int rc = ach_memcpy_h2d_async(f->dev_in[s], f->host_in[s], in_bytes, f->copy_stream);
    if (!rc) rc = ach_memcpy_h2d_async(f->dev_truth[s], f->host_truth[s], tr_bytes,
                                       f->copy_stream);
    if (!rc) rc = ach_event_record(f->copied[s], f->copy_stream);
    if (!rc) rc = ach_stream_wait_event(ns, f->copied[s]);
    if (!rc) rc = an_set_input_device(f->net, f->dev_in[s], f->dev_truth[s]);
    if (!rc) rc = ach_event_sync(f->copied[s]);
    /* the device slot is reused two batches later, after the network stream
     * has consumed it: order later copies after this device-to-device move */
    if (!rc) rc = ach_event_record(f->copied[s], ns);
    if (!rc) rc = ach_stream_wait_event(f->copy_stream, f->copied[s]);
    if (rc) return rc;
    pthread_mutex_lock(&f->mu);
    f->state[s] = SLOT_IDLE;
    start_fill(f, s, f->served + 2);
    pthread_mutex_unlock(&f->mu);
    f->served += 1;
    return ACH_OK;
}

uint64_t an_feeder_served(const an_feeder *f) { return f ? f->served : 0; }
