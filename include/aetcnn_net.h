/*
 * aetcnn_net.h -- C host layer: the reference's network and layer objects
 * (NNetwork / NLayer and its subclasses) as plain C structs with a
 * per-layer forward / backward / update function table, driving the HIP
 * kernels of aetcnn_ops.h.  Paths are relative to
 * /root/reference/src/com/ai/dnn/.
 *
 *   an_network            NNetwork (NNetwork.h:28-198)
 *   an_layer              NLayer (NLayer.h:55-196) + ConvolutionalLayer,
 *                         MaxPoolLayer, AvgPoolLayer, DropoutLayer,
 *                         SoftMaxLayer fields
 *   an_state              NetworkState (NLayer.h:21-29)
 *   an_add_*              NetworkFactory.create* (NetworkFactory.c:77-173,
 *                         543-601, 615-666)
 *   an_forward/backward   NNetwork.forward/backward (NNetwork.c:382-396,
 *                         627-654)
 *   an_update             NNetwork.updateCPU (NNetwork.c:667-680)
 *   an_train              NNetwork.train (NNetwork.c:740-758, 762-805)
 *
 * All tensors live in device memory (one arena per network); host pointers
 * appear only where a function says "host".  Functions return 0 / ACH_OK or
 * a negative ACH_E* code from aetcnn_ops.h.
 */
#ifndef AETCNN_NET_H
#define AETCNN_NET_H

#include <stddef.h>
#include <stdint.h>

#include "aetcnn_ops.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    AN_CONVOLUTIONAL = 0,
    AN_MAXPOOL = 1,
    AN_AVGPOOL = 2,
    AN_DROPOUT = 3,
    AN_SOFTMAX = 4
} an_layer_type;

typedef struct an_network an_network;
typedef struct an_layer an_layer;

/* NetworkState (NLayer.h:21-29): passed by value to every layer call. */
typedef struct {
    const float *truth;   /* device [batch][classes] one-hot, or NULL  */
    const float *input;   /* device, previous layer's output            */
    float *delta;         /* device, previous layer's delta, or NULL    */
    float *workspace;     /* device scratch shared by all layers        */
    size_t workspace_bytes;
    int train;
    int index;
} an_state;

struct an_layer {
    an_layer_type type;
    int index;
    int batch, inputs, outputs;
    int h, w, c, out_h, out_w, out_c;
    /* convolutional (ConvolutionalLayer.h:20-114) */
    int n, size, stride, pad, activation, batch_normalize, nweights;
    /* conv and maxpool: width / height strides, stride == stride_x
     * (ConvolutionalLayer.c:77-79, MaxPoolLayer.c:47-49)                    */
    int stride_x, stride_y;
    int connected;          /* an_add_connected: input read flattened       */
    float *weights, *weight_updates, *biases, *bias_updates;
    float *scales, *scale_updates;
    float *mean, *variance, *rolling_mean, *rolling_variance;
    float *mean_delta, *variance_delta;
    float *x;               /* pre-BN conv output (NormData.x)              */
    float *weights_kmajor;  /* filter layouts the conv GEMMs read, refreshed */
    float *weights_flipped; /* from weights at every forward pass            */
    /* maxpool */
    int32_t *indexes;
    /* dropout */
    float probability;
    int shares_prev;        /* output/delta alias the previous layer's    */
    /* softmax */
    int groups;
    float temperature;
    float *loss;            /* per-element cross-entropy                   */
    float *cost;            /* device scalar: sum(loss)                    */
    /* common */
    float *output, *delta;
    /* per-layer options (NLayer.h:115-125; NetworkFactory.c:656-663,
     * 926-935, 981-991): stopbackward (nonzero) ends the backward loop at this layer,
     * onlyforward skips its backward, train = 0 skips its update (set for
     * every layer below the last layer whose stopbackward is 1), learning_rate_scale
     * multiplies the rate of its update, dontload / dontloadscales /
     * flipped shape how a .weights file is read into it                   */
    int stopbackward, onlyforward, train;
    int dontload, dontloadscales, flipped;
    float learning_rate_scale;
    int zero_delta;         /* delta is accumulated into by the next layer */
    int grad_applied;       /* this step's f'(y) already applied to delta   */
    double *bias_planes;    /* conv without BN, planes of 128+ positions:
                               per-(image, filter) sums of delta, written by
                               the pass that writes delta [batch][n]     */
    int planes_ready;       /* bias_planes hold this step's sums           */
    int (*forward)(an_network *net, an_layer *l, an_state st);
    int (*backward)(an_network *net, an_layer *l, an_state st);
    int (*update)(an_network *net, an_layer *l, int batch, float lr, float momentum,
                  float decay);
};

/* ---- construction ------------------------------------------------------- */
/* Seeds the glibc rand() stream the weight init draws from
 * (WeightData.c:153-166 via DnnUtils.randUniform, DnnUtils.c:196-209).  The
 * reference initialises weights before any srand(), i.e. from seed 1.       */
void an_rand_seed(unsigned seed);
an_network *an_network_create(int batch, int h, int w, int c);
/* return the new layer's index or a negative error                          */
int an_add_convolutional(an_network *net, int filters, int size, int stride, int pad,
                         int activation, int batch_normalize);
/* Fully connected layer: the previous output flattened to inputs = c*h*w
 * features per image, weights [outputs][inputs], y = act(W x + b) or BN.
 * No counterpart in the reference's createLayer (NetworkFactory.c:615-654
 * has no CONNECTED case; the enum exists at NLayer.h:62); it follows
 * darknet's [connected] layer and runs as a 1x1 convolution of the
 * flattened input.  Init sqrt(2/inputs) * randUniform(-1,1).               */
int an_add_connected(an_network *net, int outputs, int activation, int batch_normalize);
int an_add_maxpool(an_network *net, int size, int stride, int padding);
/* The same layers with a width stride stride_x and a height stride stride_y
 * (createConvolutional / createMaxPool, NetworkFactory.c:83-90, 544-547;
 * output sizes ConvolutionalLayer.c:337-344, MaxPoolLayer.c:40-41).  A
 * convolution with unequal strides runs the reference's per-image im2col /
 * GEMM / col2im passes on the device (see ach_conv_desc.stride_y), a pool
 * the general window kernels.                                              */
int an_add_convolutional_xy(an_network *net, int filters, int size, int stride_x, int stride_y,
                            int pad, int activation, int batch_normalize);
int an_add_maxpool_xy(an_network *net, int size, int stride_x, int stride_y, int padding);
int an_add_avgpool(an_network *net);
int an_add_dropout(an_network *net, float probability);
int an_add_softmax(an_network *net, int groups, float temperature);
void an_set_hyper(an_network *net, float learning_rate, float momentum, float decay);
void an_set_dropout_seed(an_network *net, uint64_t seed);

/* Learning-rate policy: NNetwork.getCurrentRate (NNetwork.c:215-246) with
 * the [net] keys of parseNetOption (NetworkFactory.c:763-823); ids in the
 * order of the LearningRatePolicy enum (NNetwork.h:29-31).  Defaults:
 * constant, burn_in 0, power 4, gamma 1, scale 1, step 1.  steps/scales
 * (num_steps each, STEPS policy) are copied.  Rates are computed on the
 * host as the reference computes them, including its size_t arithmetic
 * (the sigmoid policy gives 0 below `step` for gamma > 0).                */
typedef enum {
    AN_POLICY_CONSTANT = 0,
    AN_POLICY_STEP = 1,
    AN_POLICY_EXP = 2,
    AN_POLICY_POLY = 3,
    AN_POLICY_STEPS = 4,
    AN_POLICY_SIG = 5,
    AN_POLICY_RANDOM = 6
} an_policy;
int an_set_policy(an_network *net, int policy, int burn_in, float power, float gamma,
                  float scale, int step, int max_batches, int num_steps, const int *steps,
                  const float *scales);
/* getCurrentRate at batch_num (host only; the random policy draws rand()) */
float an_rate(an_network *net, uint64_t batch_num);
/* the rate the next update uses: an_rate at seen / (batch * subdivisions)  */
float an_current_rate(an_network *net);
/* subdivisions (NNetwork.h:35): minibatches per update.  The network's
 * batch is the minibatch (the cfg's batch / subdivisions); an_train_step
 * runs one minibatch and updates after every subdivisions-th, with update
 * batch = batch * subdivisions (NNetwork.c:667-680, 762-805).           */
int an_set_subdivisions(an_network *net, int subdivisions);
/* The per-layer cfg options the reference's CPU path acts on (NLayer.h:
 * 115-125, read by NetworkFactory.createLayer / createNetwork,
 * NetworkFactory.c:656-663, 926-935):
 *   stopbackward        nonzero: NNetwork.backward (NNetwork.c:648) stops
 *                       before this layer's backward; exactly 1: an_finalize
 *                       also freezes every layer below the last such layer
 *                       (train = 0, onlyforward = 1; NetworkFactory.c:
 *                       887-892, 981-991)
 *   onlyforward         the backward loop skips the layer (NNetwork.c:650)
 *   learning_rate_scale the layer's update runs at rate * scale
 *                       (ConvolutionalLayer.c:960)
 *   dontload            an_load_weights skips the layer without reading its
 *                       arrays (NNetwork.c:93-94)
 *   dontloadscales      ... reads no scales / rolling mean / rolling
 *                       variance for it (ConvolutionalLayer.c:467)
 *   flipped             the weights read are transposed from [C*k*k][n] to
 *                       [n][C*k*k] (ConvolutionalLayer.c:483-485, 443-453)
 * Defaults 0 and scale 1.  Set before an_finalize (ACH_EINVAL after).    */
typedef struct {
    int stopbackward, onlyforward, dontload, dontloadscales, flipped;
    float learning_rate_scale;
} an_layer_options;
int an_set_layer_options(an_network *net, int layer, const an_layer_options *opt);
int an_get_layer_options(const an_network *net, int layer, an_layer_options *opt);
/* allocate device memory, upload initial parameters, size the workspace   */
int an_finalize(an_network *net);
void an_free(an_network *net);
/* Builds a network from a darknet-style .cfg file (ConfigFile.c:12-208,
 * NetworkFactory.c:615-1013): [net] batch/subdivisions/width/height/channels/
 * learning_rate/momentum/decay and the policy keys policy/burn_in/power/
 * step/scale/steps/scales/gamma/max_batches; [convolutional] filters/size/stride/
 * stride_x/stride_y/pad/padding/activation/batch_normalize; [connected]
 * output/activation/batch_normalize (darknet's keys, an_add_connected);
 * [maxpool] size/stride/stride_x/stride_y/padding; [avgpool]; [dropout]
 * probability; [softmax] groups/temperature; in every layer section the
 * options of an_layer_options (stopbackward, onlyforward, dontload,
 * dontloadscales, learning_rate, and flipped for [convolutional]).
 * Keys the reference reads that change its CPU training step but this
 * build does not implement (groups != 1, dilation != 1, xnor, binary,
 * bin_output, antialiasing, cbn, deformable sway / rotate / stretch,
 * assisted_excitation, share_index, maxpool_depth,
 * dropblock, softmax spatial / noloss / tree, [net] time_steps != 1) make
 * the parse fail with a message; keys the reference reads but its CPU path
 * never acts on (e.g. dontsave, clip, train_only_bn, dont_update, adam,
 * the augmentation keys) are accepted; keys the reference does not know
 * are reported on stderr as unused.  Returns NULL on error (message on
 * stderr).  The network is finalized.                                     */
an_network *an_parse_cfg(const char *path);
/* The same without an_finalize (host only: no device memory is touched);
 * the caller may inspect or change the layers, then finalizes.            */
an_network *an_parse_cfg_unfinalized(const char *path);

/* ---- darknet .weights files (NNetwork.c:64-151, ConvolutionalLayer.c:422-486)
 * header int32 {0, 2, 5} + uint64 seen, then per convolutional layer:
 * biases, [scales, rolling_mean, rolling_variance if batch_normalize],
 * weights (float32); per connected layer darknet's order: biases, weights,
 * [scales, rolling_mean, rolling_variance].  Load accepts older headers without seen and stops
 * quietly at end of file, as the reference does; it sets seen and the
 * iteration.  It honours the layer options dontload, dontloadscales and
 * flipped as NNetwork.loadWeights / ConvolutionalLayer.loadWeights do, and
 * a header whose major or minor exceeds 1000 (darknet's transposed files)
 * transposes connected layers' weights from [inputs][outputs] (darknet's
 * load_connected_weights; the reference computes this flag but loads no
 * connected layers, NNetwork.c:90).  The network must be finalized.        */
int an_save_weights(an_network *net, const char *path);
int an_load_weights(an_network *net, const char *path);

/* ---- images and their augmentation (NImage.c, ImageData.c:56-104) --------
 * an_augment holds the [net] keys of the reference's training-time
 * augmentation (parseNetOption, NetworkFactory.c:727-762), applied to every
 * image as ImageData.loadImageAugmentPaths does (ImageData.c:56-73):
 * NImage.randomAugment (NImage.c:1016-1034: aspect = randScale(aspect),
 * crop side r = randInt(min_crop, max_crop), scale = r / min(h, w*aspect),
 * rotation randUniform(-angle, angle) degrees, random offset) resampled by
 * rotateCrop (bilinear, zero outside; NImage.c:551-572), a horizontal flip
 * with probability 1/2 when flip != 0, randomDistort (hue shift
 * randUniformStrong(-hue, hue), saturation and exposure factors
 * randScale(saturation), randScale(exposure), in HSV; 3-channel images
 * only, NImage.c:201-352) and a bilinear resize back to the input size
 * (NImage.c:474-530).  Random numbers: the counter-based hash of
 * an_feeder_sample(seed, batch_no, image, salt), one salt per draw, through
 * the reference's formulas with RAND_MAX = 2^31 - 1.                       */
typedef struct {
    int min_crop, max_crop;     /* crop side range; defaults w and 2*w       */
    float angle;                /* degrees; default 0                        */
    float aspect;               /* default 1                                 */
    float hue;                  /* default 0                                 */
    float saturation, exposure; /* defaults 1                                */
    int flip;                   /* default 1                                 */
} an_augment;
void an_augment_defaults(an_augment *a, int net_w);
/* the augmentation keys and label_smooth_eps of a .cfg's [net] section    */
int an_cfg_augment(const char *cfg_path, an_augment *a, float *label_smooth_eps);
/* one image of batch batch_no: src and dst are host [c][h][w] planes       */
int an_augment_image(const float *src, int w, int h, int c, const an_augment *a, uint64_t seed,
                     uint64_t batch_no, int image, float *dst);
/* the steps, host-only: rotateCrop (rad, scale s, output w x h, offset dx,
 * dy, aspect), flip, distort (HSV; 3 channels), resizeImage               */
void an_image_rotate_crop(const float *src, int W, int H, int c, float rad, float s, int w, int h,
                          float dx, float dy, float aspect, float *dst);
void an_image_flip(float *im, int w, int h, int c);
void an_image_distort(float *im, int w, int h, float hue, float sat, float val);
/* resizeImage returns ACH_EINVAL (dst unwritten) for a bad size or when
 * its row buffer cannot be allocated                                       */
int an_image_resize(const float *src, int W, int H, int c, int w, int h, float *dst);
/* NImage.reload (NImage.c:638-658): decodes a PNG (8-bit, non-interlaced;
 * grey, RGB, palette, grey+alpha, RGBA), a baseline / extended sequential
 * JPEG (greyscale, YCbCr or Adobe RGB; any sampling; restart intervals) or
 * a binary PPM / PGM file into host planes dst[c][h][w] = sample / 255; the
 * file must have exactly w x h pixels and c channels (else ACH_EINVAL with a
 * message).  The reference decodes through stb_image; progressive,
 * arithmetic-coded, 12-bit and CMYK JPEG and other formats are refused.    */
int an_image_load(const char *path, int w, int h, int c, float *dst);
/* NImage.createImage (NImage.c:587-610): decodes a file at its own size
 * into *dst = malloc'd planes [c][*h][*w] (free with an_image_free), with
 * c (1-4) channels whatever the file holds, converted as stb_image does
 * when the reference asks for a channel count: grey replicated, alpha
 * dropped or opaque, RGB to grey as (77 r + 150 g + 29 b) >> 8.           */
int an_image_read(const char *path, int c, int *w, int *h, float **dst);
void an_image_free(float *im);
/* NImage.resizeMin (NImage.c:1037-1051): the w x h whose smaller side is
 * min (integer scaling of the other side); NImage.crop (NImage.c:439-458):
 * the w x h window at (dx, dy) with coordinates clamped into the image     */
void an_image_resize_min_size(int W, int H, int min, int *w, int *h);
void an_image_crop(const float *src, int W, int H, int c, int dx, int dy, int w, int h,
                   float *dst);
/* ImageData.fillTruthSmooth (ImageData.c:80-104): the index of the one
 * label that occurs in path as a substring, or -1 for none or several     */
int an_label_from_path(const char *path, const char *const *labels, int nlabels);

/* ---- validation (Classifier.validateSingle, Classifier.c:359-464) ---------
 * For every path of list_file: its class is the first label that occurs in
 * it (-1, a miss, when none does); the image is read at its own size with
 * the network's channel count, resized so its smaller side is the network
 * width, cut to the network's w x h around its centre
 * (an_validation_image), predicted (an_predict, the images filling the
 * network's batch; a last partial batch padded with zero images) and its
 * topk best classes taken (an_top_k; topk is clamped to the classes).
 * top1_accuracy / topk_accuracy: the fraction of images whose class is the
 * best / among the topk best.  The reference predicts one image at a time
 * on a batch-1 network; inference is per image, so batching it changes
 * only the rounding of the convolutions' sums.                              */
typedef struct {
    int images, unlabeled, topk;
    float top1_accuracy, topk_accuracy;
} an_validation;
int an_validate_paths(an_network *net, const char *list_file, const char *const *labels,
                      int nlabels, int topk, an_validation *result);
int an_validation_image(const char *path, int w, int h, int c, float *dst);

/* ---- input pipeline (ImageData.c:20-224, DstbCompute.c:60-216) ------------
 * Worker threads fill two pinned host batches; an_feeder_next copies the next
 * one to the device on the feeder's own stream (overlapping the previous
 * training step), orders the network's stream after it and makes it the
 * network's input and truth.  Image i of batch k is drawn from a counter-
 * based hash of (seed, k, i): an_feeder_sample(seed, k, i, 0) % (number of
 * images) is its index.  Truth is one-hot with label smoothing
 * (fillTruthSmooth, ImageData.c:77-103).  Sources:
 *   paths     a list file of image paths, one per line (the reference's
 *             training list, Classifier.c:79-108), decoded by an_image_load,
 *             labels from path substrings (an_label_from_path, checked for
 *             the whole list at creation; labels[nlabels], nlabels = the
 *             network's classes)
 *   cifar     CIFAR-10 binary batches (1 label byte + 3x32x32 planar RGB
 *             bytes per record; pixels / 255); needs a 3x32x32 input
 *   synthetic pixels uniform in [0,1) (an_feeder_sample(seed, k,
 *             i*inputs + j, 2) >> 40 / 2^24), labels an_feeder_sample(seed,
 *             k, i, 3) % classes
 * With aug != NULL every image then takes an_augment_image(seed, k, i);
 * NULL feeds the images as decoded.  an_feeder_next returns ACH_EINVAL when
 * an image could not be decoded (the reference aborts).  Free the feeder
 * before the network.                                                     */
typedef struct an_feeder an_feeder;
an_feeder *an_feeder_create_paths(an_network *net, const char *list_file,
                                  const char *const *labels, int nlabels, int threads,
                                  uint64_t seed, const an_augment *aug, float label_smooth_eps);
an_feeder *an_feeder_create_cifar(an_network *net, const char *const *files, int nfiles,
                                  int threads, uint64_t seed, const an_augment *aug,
                                  float label_smooth_eps);
an_feeder *an_feeder_create_synthetic(an_network *net, int threads, uint64_t seed,
                                      const an_augment *aug);
int an_feeder_next(an_feeder *f);
uint64_t an_feeder_served(const an_feeder *f);
uint64_t an_feeder_sample(uint64_t seed, uint64_t batch_no, int image, int what);
void an_feeder_free(an_feeder *f);

/* ---- training ------------------------------------------------------------- */
ach_stream_t an_stream(an_network *net);
/* copy one batch from host buffers into the network's input/truth        */
int an_set_input(an_network *net, const float *host_input, const float *host_truth);
/* the same from device buffers (device-to-device copy on the net stream) */
int an_set_input_device(an_network *net, const float *dev_input, const float *dev_truth);
/* One minibatch of NNetwork.train (NNetwork.c:740-805) on the resident
 * input: seen += batch, forward, backward, and after every
 * subdivisions-th minibatch cur_iteration += 1 and the update.  Enqueues
 * on the network's stream and returns without synchronising; the loss
 * stays on the device until an_get_loss.  Dropout masks use the index
 * seen/batch of the minibatch (before the increment) as their step.       */
int an_train_step(an_network *net);
/* synchronises and returns sum(cost)/batch of the last minibatch (the
 * reference returns the mean of these over the subdivisions, NNetwork.c:804).
 * Returns ACH_ENAN, with a message on stderr, where the reference's CPU path
 * stops on a NaN: a NaN loss, or a NaN that a training step left in a
 * batch-norm layer's mean or variance (NormData.normalize exits on a NaN
 * normalized value, NormData.c:273-276) or in its scales or scale updates
 * (ScaleData.c:51-54, 67-70).  Every step ends with one scan of those arrays
 * (ach_nan_scan); the finding is sticky, as the state then holds the NaN.  */
int an_get_loss(an_network *net, float *loss);
/* synchronises; 0 while no step has left a NaN in those arrays, else 1 with
 * *layer the first such layer and *what 0 mean, 1 variance, 2 scales,
 * 3 scale updates.  No counterpart in the reference (it exits instead).   */
int an_nan_status(an_network *net, int *layer, int *what);
/* host-buffer convenience: set_input + train_step + get_loss               */
int an_train(an_network *net, const float *host_input, const float *host_truth, float *loss);
int an_forward(an_network *net, int train);
/* NNetwork.predict (NNetwork.c:411-422): inference forward on a host batch
 * (batch-norm on the rolling statistics, dropout off, no truth); copies the
 * last layer's output, batch x outputs floats, to host_output.              */
int an_predict(an_network *net, const float *host_input, float *host_output);
/* NNetwork.fuseConvBatchnorm (NNetwork.c:272-288): fold every batch-norm conv
 * layer's inference BN into its filters and biases (ach_conv_bn_fold) and
 * make it a plain conv layer with bias; synchronous.  Used before inference
 * (Classifier.c:369-373).                                                   */
int an_fuse_conv_batchnorm(an_network *net);
/* DnnUtils.topK (DnnUtils.c:463-477): the k largest of a[0..n), largest
 * first (ties ordered as the reference's strict-'>' insertion leaves them);
 * host-only                                                                 */
void an_top_k(const float *a, int n, int k, int *index);
int an_backward(an_network *net);
int an_update(an_network *net);
/* one layer with the NetworkState the loops above would give it
 * (NLayer.forward / NLayer.backward, NLayer.h:159-166)                     */
int an_layer_forward(an_network *net, int layer, int train);
int an_layer_backward(an_network *net, int layer);

/* ---- introspection (tests, checkpoints) ------------------------------------ */
int an_n_layers(const an_network *net);
an_layer *an_get_layer(an_network *net, int i);
/* out[8] = {type, out_c, out_h, out_w, c, h, w, batch}; host-only, valid
 * before an_finalize                                                        */
int an_layer_shape(const an_network *net, int i, int *out8);
int an_batch(const an_network *net);
/* device pointers of the network's input and truth buffers                 */
float *an_input(an_network *net);
float *an_truth(an_network *net);
int an_classes(const an_network *net);
uint64_t an_seen(const an_network *net);
int an_iteration(const an_network *net);
/* device buffer of a layer: which = 0 output, 1 delta, 2 weights,
 * 3 weight_updates, 4 biases, 5 bias_updates, 6 scales, 7 scale_updates,
 * 8 rolling_mean, 9 rolling_variance, 10 mean, 11 variance, 12 x (pre-BN),
 * 14 indexes (int32), 15 loss; *count = elements (0 if absent)              */
void *an_layer_buffer(an_network *net, int layer, int which, size_t *count);
/* total GFLOP of one training step's conv GEMMs (fwd + wgrad + dgrad where
 * the layer has an input gradient)                                          */
double an_step_conv_gflop(const an_network *net);

#ifdef __cplusplus
}
#endif
#endif
