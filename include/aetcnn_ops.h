/*
 * aetcnn_ops.h -- C-ABI of the MI355X (gfx950) HIP kernels for one CNN
 * training step of aet-cnn.  Plain pointers and sizes only; every pointer
 * argument named like a tensor is DEVICE memory unless stated otherwise.
 *
 * Each entry point replaces one operation of the reference's CPU path
 * (paths relative to /root/reference/src/com/ai/dnn/) with CPU-path
 * semantics; the reference's own GPU ("mtcs") path differs from its CPU path
 * (biased BN variance, other eps, 0.99 rolling momentum, beta gradient) and
 * is NOT what these functions compute.
 *
 * Conventions
 *  - tensors are fp32 NCHW, batch outermost: ((b*C + c)*H + h)*W + w
 *  - `stream` is a hipStream_t passed as void*; NULL = the null stream
 *  - functions return 0 on success or a negative ACH_E* code; nothing is
 *    synchronised unless the name says so
 *  - functions that need scratch take (ws, ws_bytes) and have a matching
 *    *_workspace() query; kernels never allocate
 */
#ifndef AETCNN_OPS_H
#define AETCNN_OPS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ACH_OK 0
#define ACH_EINVAL (-1)     /* bad argument / shape                        */
#define ACH_EWORKSPACE (-2) /* workspace missing or too small               */
#define ACH_EHIP (-3)       /* HIP runtime error (ach_last_hip_error())     */
#define ACH_EUNSUPPORTED (-4)
#define ACH_ENAN (-5)       /* a NaN where the reference's CPU path exits    */

/* Activation ids = the reference's ActivationType order (Activation.h). */
#define ACH_LOGISTIC 0
#define ACH_RELU 1
#define ACH_LINEAR 3
#define ACH_LEAKY 7

typedef void *ach_stream_t;

/* ---- runtime plumbing (the reference's MtcsMem / MtcsStream roles:
 *      mtcs/MtcsTool.c:22-30, mtcs/MtcsData.c:20-28) ----------------------- */
const char *ach_version(void);
int ach_device_count(void);
int ach_set_device(int dev);
const char *ach_last_hip_error(void);
int ach_malloc(void **ptr, size_t bytes);
int ach_free(void *ptr);
int ach_host_alloc(void **ptr, size_t bytes); /* pinned host memory */
int ach_host_free(void *ptr);
int ach_memcpy_h2d(void *dst, const void *src, size_t bytes, ach_stream_t stream);
int ach_memcpy_d2h(void *dst, const void *src, size_t bytes, ach_stream_t stream);
int ach_memcpy_d2d(void *dst, const void *src, size_t bytes, ach_stream_t stream);
/* enqueue only (no synchronisation); truly asynchronous from pinned memory */
int ach_memcpy_h2d_async(void *dst, const void *src, size_t bytes, ach_stream_t stream);
int ach_stream_create(ach_stream_t *stream);
int ach_stream_destroy(ach_stream_t stream);
int ach_stream_sync(ach_stream_t stream);
int ach_device_sync(void);
/* events for timing (hipEvent_t as void*) */
int ach_event_create(void **ev);
int ach_event_destroy(void *ev);
int ach_event_record(void *ev, ach_stream_t stream);
int ach_event_elapsed_ms(void *start, void *stop, float *ms); /* syncs stop */
int ach_event_sync(void *ev);                         /* host waits for ev */
int ach_stream_wait_event(ach_stream_t stream, void *ev); /* stream waits for ev */

/* ---- BLAS-1 helpers (mtcs/MtcsTool.c:33-132; NData.setZero NData.c:232) */
int ach_fill(float *x, size_t n, float value, ach_stream_t stream);
int ach_axpy(size_t n, float alpha, const float *x, float *y, ach_stream_t stream);
int ach_scal(size_t n, float alpha, float *x, ach_stream_t stream);

/* ---- GEMM (Gemm.gemm, Gemm.c:116-144; Gemm.h:12-16) --------------------
 * Row-major C = ALPHA*op(A)*op(B) + BETA*C on fp32 MFMA.                  */
int ach_gemm(int TA, int TB, int M, int N, int K, float ALPHA,
             const float *A, int lda, const float *B, int ldb,
             float BETA, float *C, int ldc, ach_stream_t stream);

/* ---- im2col / col2im for one image (Im2Col.c:65-103, 155-192; the
 * signatures of Im2Col.h:10-15, 24-28, dilation included: window taps at
 * k*dilation, output size (in + 2*pad - (dilation*(k-1)+1))/stride + 1).
 * Dilation below 1 returns ACH_EINVAL.  (The conv entry points below take
 * no dilation: the cfg parser rejects dilated convolutions.)              */
int ach_im2col(const float *im, int channels, int height, int width,
               int kh, int kw, int ph, int pw, int sh, int sw,
               int dilation_h, int dilation_w, float *col, ach_stream_t stream);
/* col2im zeroes `im` first, as the reference does (Im2Col.c:162)          */
int ach_col2im(const float *col, int channels, int height, int width,
               int kh, int kw, int ph, int pw, int sh, int sw,
               int dilation_h, int dilation_w, float *im, ach_stream_t stream);

/* ---- convolution (ConvolutionalLayer.c:684-803, 906-947) ----------------
 * stride is the width stride (the layer's stride_x, ConvolutionalLayer.c:
 * 77-79) and stride_y the height stride, 0 meaning the same as stride; the
 * output is ((h + 2*pad - size)/stride_y + 1) x ((w + 2*pad - size)/stride
 * + 1) (ConvolutionalLayer.c:337-344).  With unequal strides every entry
 * point below runs the reference's per-image passes on the device -- the
 * forward im2col + GEMM (ConvolutionalLayer.c:790-803), the weight
 * gradient im2col + GEMM added into dw and the input gradient GEMM +
 * col2im (:913-945) -- with one image's column buffer as workspace, except
 * for a fully connected geometry (one output position, which no stride
 * moves), and ach_conv_bwd_data_prepared returns ACH_EUNSUPPORTED.       */
typedef struct {
    int batch, c, h, w;   /* input  [batch][c][h][w]                     */
    int n;                /* filters (output channels)                   */
    int size, stride, pad;/* square kernel, stride, padding (groups = 1) */
    int stride_y;         /* height stride; 0: the same as stride        */
} ach_conv_desc;

int ach_conv_out_h(const ach_conv_desc *d);
int ach_conv_out_w(const ach_conv_desc *d);
/* y = W * im2col(x), overwriting y        (ConvolutionalLayer.c:689,716-803) */
size_t ach_conv_fwd_workspace(const ach_conv_desc *d);
int ach_conv_fwd(const ach_conv_desc *d, const float *x, const float *w, float *y,
                 void *ws, size_t ws_bytes, ach_stream_t stream);
/* dx = col2im(W^T * dy), overwriting dx   (ConvolutionalLayer.c:933-945)   */
size_t ach_conv_bwd_data_workspace(const ach_conv_desc *d);
int ach_conv_bwd_data(const ach_conv_desc *d, const float *dy, const float *w, float *dx,
                      void *ws, size_t ws_bytes, ach_stream_t stream);
/* dw += sum_b dy_b * im2col(x_b)^T        (ConvolutionalLayer.c:913-929)   */
size_t ach_conv_bwd_filter_workspace(const ach_conv_desc *d);
int ach_conv_bwd_filter(const ach_conv_desc *d, const float *x, const float *dy, float *dw,
                        void *ws, size_t ws_bytes, ach_stream_t stream);
/* ach_conv_bwd_filter, then the weights' step of ConvolutionalLayer.update
 * (ConvolutionalLayer.c:959-980) on (w, dw): dw += decay_coef*w;
 * w += lr_coef*dw; dw *= momentum -- the results of ach_conv_bwd_filter
 * followed by ach_sgd_update(F*C*k*k, w, dw, ...), bit for bit, with the
 * update done in the pass that finishes dw (no pass of its own).  The
 * caller orders it after every reader of w: ach_conv_bwd_data_reads_w(d)
 * tells whether this layer's _prepared input gradient is one.  Same
 * workspace as ach_conv_bwd_filter.                                       */
int ach_conv_bwd_filter_sgd(const ach_conv_desc *d, const float *x, const float *dy, float *w,
                            float *dw, float decay_coef, float lr_coef, float momentum, void *ws,
                            size_t ws_bytes, ach_stream_t stream);
/* 1 if ach_conv_bwd_data_prepared (or ach_conv_bwd_data) reads w, 0 if it
 * reads only the flipped copy wft (stride 1, filters wider than 1x1, more
 * than 4 input channels)                                                   */
int ach_conv_bwd_data_reads_w(const ach_conv_desc *d);

/* ---- prepared filters -------------------------------------------------------
 * The conv GEMMs read the filter k-major (Wt[C*k*k][n]) and, for the stride-1
 * input gradient, flipped k-major (Wft[(f*k*k + t)*C + c] = W[f][c][k*k-1-t]).
 * ach_conv_fwd / ach_conv_bwd_data build these in the workspace on every
 * call; a caller that keeps them (the network refreshes all of them with one
 * ach_conv_prepare_filters launch per step) calls the _prepared variants.
 * wft may be NULL when not needed: stride > 1, or a 1x1 filter (including a
 * kernel covering the whole unpadded input), whose flipped copy is W itself.
 * A fully connected geometry (ach_conv_is_fully_connected: a kernel covering
 * the whole unpadded input, or a 1x1 filter on a 1x1 input) needs no copy at
 * all: ach_conv_prepare_filters leaves its wt untouched and the _prepared
 * forward reads its wt argument as the filter itself, so pass w there.
 * No counterpart in the reference, which has no such layouts.              */
typedef struct {
    ach_conv_desc desc;
    const float *w;   /* [n][c][size][size] */
    float *wt;        /* n*c*size*size floats */
    float *wft;       /* n*c*size*size floats or NULL */
} ach_filter_job;
int ach_conv_prepare_filters(int njobs, const ach_filter_job *jobs, ach_stream_t stream);
/* 1 for a fully connected geometry (see above), else 0                    */
int ach_conv_is_fully_connected(const ach_conv_desc *d);
/* workspace: ach_conv_fwd_workspace(d) / ach_conv_bwd_data_workspace(d)
 * bytes suffice (the _prepared calls use only the split-K part of it)      */
int ach_conv_fwd_prepared(const ach_conv_desc *d, const float *x, const float *wt, float *y,
                          void *ws, size_t ws_bytes, ach_stream_t stream);
/* The forward of a convolutional layer without batch-norm in one pass:
 * y = act(conv(x) + bias), the output-side steps of ConvolutionalLayer.
 * forward (ConvolutionalLayer.c:684-716, then IOData.addBias IOData.c:43-55
 * and activate IOData.c:60-72) applied to each sum in the GEMM epilogue
 * (or the split-K reduction) with the same fp32 arithmetic: the results
 * are those of ach_conv_fwd_prepared + ach_add_bias + ach_activate, bit for
 * bit.  bias may be NULL (no bias); activation is ACH_LOGISTIC, ACH_RELU,
 * ACH_LINEAR or ACH_LEAKY (else ACH_EUNSUPPORTED); the logistic activation
 * (a double exp per element) and, for 256-row tiles without a K split,
 * bias and activation run as separate passes inside the call.             */
int ach_conv_fwd_bias_act_prepared(const ach_conv_desc *d, const float *x, const float *wt,
                                   const float *bias, int activation, float *y, void *ws,
                                   size_t ws_bytes, ach_stream_t stream);
/* stride-1 only (ACH_EUNSUPPORTED otherwise); w is read for 1x1 filters,
 * wft otherwise                                                             */
int ach_conv_bwd_data_prepared(const ach_conv_desc *d, const float *dy, const float *w,
                               const float *wft, float *dx, void *ws, size_t ws_bytes,
                               ach_stream_t stream);

/* ---- bias (IOData.addBias IOData.c:43-55; BiasData.calcGrad BiasData.c:40-57) */
int ach_add_bias(float *out, const float *biases, int batch, int n, int spatial,
                 ach_stream_t stream);
/* bias_updates[c] += sum of delta over images and positions; the workspace
 * (ach_bias_grad_workspace bytes) holds double partial sums per image chunk */
size_t ach_bias_grad_workspace(int batch, int n, int spatial);
int ach_bias_grad(float *bias_updates, const float *delta, int batch, int n, int spatial,
                  void *ws, size_t ws_bytes, ach_stream_t stream);
/* The same gradient in two halves, for a pass that already writes the delta
 * (the activation gradient below, or a max-pool's input gradient): that
 * pass stores plane_sums[b][c] = sum over positions of delta[b][c][:]
 * (double [batch][n]: DnnUtils.sum of each image's plane, BiasData.c:
 * 52-56), and this call adds bias_updates[c] += sum over b ascending of
 * plane_sums[b][c] (in double, rounded once).                             */
int ach_bias_grad_planes(float *bias_updates, const double *plane_sums, int batch, int n,
                         ach_stream_t stream);

/* ---- batch-norm, training mode ------------------------------------------
 * Forward (forwardNormCPU NLayer.c:141-162 = NormData.calcVarianceAndMean
 * NormData.c:141-186, scalAxpyRollMeanAndRollVariance :224-229, normalize
 * :244-282).  `out` holds the conv output on entry; on return x = copy of it,
 * x_norm (optional, may be NULL) = (x-mean)/(sqrt(var)+1e-6), and
 * out = act(x_norm*scales + biases) where act is ACH_LINEAR for the plain op
 * or ACH_LEAKY / ACH_RELU to fuse the layer's activation (Activation.c:160).
 * mean/variance (unbiased) and rolling_mean/rolling_variance (.9/.1) are
 * updated.  `x` may equal NULL only if x_norm is also NULL and the caller
 * keeps the pre-BN tensor itself (pass it as `out` != x is required).        */
size_t ach_bn_workspace(int batch, int c, int spatial);
int ach_bn_train_fwd(float *out, int batch, int c, int spatial,
                     const float *scales, const float *biases,
                     float *mean, float *variance,
                     float *rolling_mean, float *rolling_variance,
                     float *x, float *x_norm, int activation,
                     void *ws, size_t ws_bytes, ach_stream_t stream);
/* Same, reading the pre-BN tensor from `x` and writing only `out`
 * (x is not copied): the layout the network driver uses.                   */
int ach_bn_train_fwd_from_x(const float *x, float *out, int batch, int c, int spatial,
                            const float *scales, const float *biases,
                            float *mean, float *variance,
                            float *rolling_mean, float *rolling_variance,
                            int activation, void *ws, size_t ws_bytes,
                            ach_stream_t stream);
/* Allocation-free variant of ach_bn_train_fwd_from_x.  No counterpart in
 * the reference: it is for callers that cannot allocate or pass scratch
 * memory (work recorded into a HIP graph, tight serving loops, harnesses
 * that forbid hipMalloc).  The per-(channel, image chunk) partial sums go to
 * a fixed device array of ACH_BN_NOALLOC_SCRATCH_BYTES that the library
 * holds on each device it runs on until the process ends; the call makes no
 * allocation of any kind.  Same arguments and results as
 * ach_bn_train_fwd_from_x without (ws, ws_bytes).  Limit: the partial sums
 * (ach_bn_workspace(batch, c, spatial) bytes) must fit the array, which
 * holds every shape with c <= 10922 channels; larger shapes return
 * ACH_EWORKSPACE with a message in ach_last_hip_error().  Every call on one
 * device shares that device's array: calls that overlap in time on one
 * device (e.g. on two streams) race and must be ordered by the caller.    */
#define ACH_BN_NOALLOC_SCRATCH_BYTES (256u * 1024u)
int ach_bn_train_fwd_from_x_noalloc(const float *x, float *out, int batch, int c, int spatial,
                                    const float *scales, const float *biases,
                                    float *mean, float *variance,
                                    float *rolling_mean, float *rolling_variance,
                                    int activation, ach_stream_t stream);
/* Inference (forwardNormCPU test branch, NLayer.c:155-160 ->
 * NormData.normalizeByRoll, NormData.c:291-326): out = act(((x - rolling_mean)
 * * inv) * scales + biases), inv = 1/(sqrt(rolling_variance) + 1e-6) in
 * double; statistics are not updated.  x may equal out.                    */
int ach_bn_infer(const float *x, float *out, int batch, int c, int spatial,
                 const float *scales, const float *biases, const float *rolling_mean,
                 const float *rolling_variance, int activation, ach_stream_t stream);
/* Conv-BN folding for inference (ConvolutionalLayer.fuseConvBatchnorm,
 * ConvolutionalLayer.c:983-1003): per filter f, r = sqrt((double)
 * rolling_variance[f] + 1e-5); biases[f] -= scales[f]*rolling_mean[f]/r and
 * weights[f][0..fsize) *= scales[f]/r, in double, rounded once to float.
 * weights is [filters][fsize] (fsize = C*k*k), updated in place.           */
int ach_conv_bn_fold(int filters, int fsize, float *weights, float *biases,
                     const float *scales, const float *rolling_mean,
                     const float *rolling_variance, ach_stream_t stream);
/* Backward (backwardNormCPU NLayer.c:246-278): scale_updates += sum(d*x_norm);
 * d *= scales; mean_delta, variance_delta; d <- normalize_delta.  No beta
 * gradient (the CPU path computes none).  If activation is ACH_LEAKY/RELU the
 * activation gradient (ConvolutionalLayer.c:898, Activation.c:233-239) is
 * applied to `delta` first, its sign taken from the recomputed BN output.
 * x_norm may be NULL (recomputed from x).  mean_delta/variance_delta may be
 * NULL.                                                                     */
int ach_bn_bwd(float *delta, int batch, int c, int spatial,
               const float *x, const float *x_norm,
               const float *mean, const float *variance,
               const float *scales, const float *biases, float *scale_updates,
               float *mean_delta, float *variance_delta, int activation,
               void *ws, size_t ws_bytes, ach_stream_t stream);

/* ---- activations (Activation.c:160-179 activate, :233-239 gradientArray) */
int ach_activate(float *x, size_t n, int activation, ach_stream_t stream);
int ach_gradient(const float *y, size_t n, int activation, float *delta,
                 ach_stream_t stream);
/* ach_gradient of a [batch][n][spatial] tensor (the same products, ACH_LINEAR
 * included: delta unchanged) that also stores the bias gradient's
 * plane_sums[b][c] of the result (ach_bias_grad_planes)                    */
int ach_gradient_planes(const float *y, int batch, int n, int spatial, int activation,
                        float *delta, double *plane_sums, ach_stream_t stream);

/* ---- max-pool (MaxPoolLayer.c:237-272 forward, :318-331 backward) --------
 * out size = (in + padding - size)/stride + 1, window offset -padding/2,
 * -FLT_MAX init, strict '>' (first max in row-major scan wins); indexes are
 * global flat input indices.  Backward adds into delta_in in ascending
 * output order, bit-identical to the reference's scatter loop.  With
 * accumulate = 0 the sums start from +0 instead of delta_in's contents (the
 * reference's delta is zeroed in forward, NNetwork.c:388-391), so a caller
 * whose delta_in is all zeros may skip that zeroing; delta_in is then only
 * written.                                                                 */
int ach_maxpool_out(int in, int size, int stride, int padding);
int ach_maxpool_fwd(const float *in, int batch, int c, int h, int w,
                    int size, int stride, int padding,
                    float *out, int32_t *indexes, ach_stream_t stream);
int ach_maxpool_bwd(const float *delta_out, const int32_t *indexes,
                    int batch, int c, int h, int w, int size, int stride, int padding,
                    float *delta_in, int accumulate, ach_stream_t stream);
/* The same pool with a width stride stride_x and a height stride stride_y
 * (MaxPoolLayer.c:40-41, 255-256: out w = (w + padding - size)/stride_x + 1,
 * h likewise with stride_y); equal strides take the calls above.           */
int ach_maxpool_fwd_xy(const float *in, int batch, int c, int h, int w, int size, int stride_x,
                       int stride_y, int padding, float *out, int32_t *indexes,
                       ach_stream_t stream);
int ach_maxpool_bwd_xy(const float *delta_out, const int32_t *indexes, int batch, int c, int h,
                       int w, int size, int stride_x, int stride_y, int padding, float *delta_in,
                       int accumulate, ach_stream_t stream);
/* A dropout layer that follows the max-pool and shares its output
 * (DropoutLayer.c:55-86, NetworkFactory.c:644-650), applied by the pool:
 * the forward writes the masked output (ach_maxpool_fwd + ach_dropout_fwd on
 * out), the backward masks delta_out as it reads it (ach_dropout_bwd on
 * delta_out + ach_maxpool_bwd; delta_out itself may be left unmasked) --
 * the same values bit for bit.  Fused into the 2x2 / stride
 * 2 kernels; other windows run the two steps inside the call.  (The network
 * loops of aetcnn_net.h run pool and dropout as separate layers, as the
 * reference does, so the shared delta is masked in place.)                */
int ach_maxpool_fwd_dropout(const float *in, int batch, int c, int h, int w,
                            int size, int stride, int padding, float *out, int32_t *indexes,
                            float probability, uint64_t seed, uint32_t iter, uint32_t layer,
                            ach_stream_t stream);
int ach_maxpool_bwd_dropout(float *delta_out, const int32_t *indexes,
                            int batch, int c, int h, int w, int size, int stride, int padding,
                            float *delta_in, int accumulate, float probability, uint64_t seed,
                            uint32_t iter, uint32_t layer, ach_stream_t stream);
/* ach_maxpool_bwd, then delta_in *= f'(y_in) with the previous layer's
 * output y_in and activation act_in (Activation.gradientArray,
 * Activation.c:233-239, the first step of that layer's backward,
 * ConvolutionalLayer.c:863-948) in the same pass: the same values, bit for
 * bit, as ach_maxpool_bwd + ach_gradient.  Used when the pool's input
 * gradient is that layer's whole delta.                                   */
int ach_maxpool_bwd_act(const float *delta_out, const int32_t *indexes,
                        int batch, int c, int h, int w, int size, int stride, int padding,
                        float *delta_in, int accumulate, const float *y_in, int act_in,
                        ach_stream_t stream);
/* ach_maxpool_bwd_act with accumulate = 0 (y_in may be NULL: no gradient)
 * that also stores the bias gradient's plane_sums[b][c] of the delta_in it
 * writes (ach_bias_grad_planes; double [batch][c]).  For pools whose output
 * planes are staged in LDS with at most 8 planes per workgroup (input
 * planes of 128+ pixels, output planes of at most 4096): ACH_EUNSUPPORTED
 * otherwise, with nothing launched.                                       */
int ach_maxpool_bwd_act_planes(const float *delta_out, const int32_t *indexes, int batch, int c,
                               int h, int w, int size, int stride, int padding, float *delta_in,
                               const float *y_in, int act_in, double *plane_sums,
                               ach_stream_t stream);
/* ach_maxpool_bwd_act_planes (plane_sums may be NULL here) for a relu or
 * leaky layer below, with the activation gradient taken from the pool's
 * own forward output `pooled` instead of the layer's output: a pixel that
 * receives a sum is the argmax of its windows and the window's output is
 * its value, so the results equal ach_maxpool_bwd_act_planes' bit for bit
 * while reading the pooled tensor instead of the pool's input.  `pooled`
 * must hold what ach_maxpool_fwd wrote (not masked in place since).
 * ACH_EINVAL for another activation; ACH_EUNSUPPORTED, with nothing
 * launched, for pools the plane-staged kernel does not take (as above).   */
int ach_maxpool_bwd_act_pooled(const float *delta_out, const int32_t *indexes, int batch, int c,
                               int h, int w, int size, int stride, int padding, float *delta_in,
                               const float *pooled, int act_in, double *plane_sums,
                               ach_stream_t stream);

/* ---- global average pool (AvgPoolLayer.c:29-46, 73-88) ----------------- */
int ach_avgpool_fwd(const float *in, int batch, int c, int spatial, float *out,
                    ach_stream_t stream);
int ach_avgpool_bwd(const float *delta_out, int batch, int c, int spatial,
                    float *delta_in, ach_stream_t stream);

/* ---- softmax + cross-entropy (SoftMaxLayer.c:47-119) ---------------------
 * output = softmax(in/temperature) per (image, group); if truth != NULL:
 * error = t ? -log(p) : 0, delta = t - p, *cost (device float) = sum(error).
 * Backward is ach_axpy(n, 1, delta, delta_prev) (SoftMaxLayer.c:313).      */
size_t ach_softmax_workspace(int batch, int groups);
int ach_softmax_xent(const float *in, int batch, int inputs, int groups,
                     float temperature, const float *truth,
                     float *output, float *delta, float *error, float *cost,
                     void *ws, size_t ws_bytes, ach_stream_t stream);

/* ---- dropout (DropoutLayer.c:55-86) ---------------------------------------
 * r = u(seed, iter, layer, i) from a counter-based generator (SplitMix64
 * finaliser, top 24 bits); r < p -> 0 else x * 1/(1-p).  Same mask forward
 * and backward; nothing is stored.                                          */
float ach_dropout_uniform(uint64_t seed, uint32_t iter, uint32_t layer, uint32_t i);
int ach_dropout_fwd(float *x, size_t n, float probability, uint64_t seed,
                    uint32_t iter, uint32_t layer, ach_stream_t stream);
int ach_dropout_bwd(float *delta, size_t n, float probability, uint64_t seed,
                    uint32_t iter, uint32_t layer, ach_stream_t stream);

/* ---- NaN scan (the reference's isnan checks: NormData.normalize exits on a
 * NaN normalized value, NormData.c:273-276; ScaleData.addUpdatesToScale and
 * scaleUpdates abort on a NaN scale or scale update, ScaleData.c:51-54,
 * 67-70).  spans (device memory) lists nspans arrays; for every array that
 * holds a NaN, *flag = min(*flag, its tag), so with tags in checking order
 * *flag names the first offending array.  One launch for all the arrays;
 * the caller initialises *flag (e.g. to INT32_MAX) and reads it later.     */
typedef struct ach_nan_span {
    const float *p;
    uint64_t n;
    int32_t tag;
    int32_t reserved;
} ach_nan_span;
int ach_nan_scan(const ach_nan_span *spans, int nspans, int32_t *flag, ach_stream_t stream);

/* ---- SGD momentum / weight-decay update ----------------------------------
 * ConvolutionalLayer.update (ConvolutionalLayer.c:959-980):
 *   dW += -decay*batch*W; W += (lr/batch)*dW; dW *= momentum;
 *   b  += (lr/batch)*db;  db *= momentum;  (scales likewise, no decay)
 * scales/scale_updates may be NULL.                                        */
int ach_conv_update(size_t nweights, float *weights, float *weight_updates,
                    size_t n, float *biases, float *bias_updates,
                    float *scales, float *scale_updates,
                    int batch, float learning_rate, float momentum, float decay,
                    ach_stream_t stream);
/* One flat buffer: v += decay_coef*w; w += lr_coef*v; v *= momentum, with
 * decay_coef = -decay*batch (0 for no decay), lr_coef = lr/batch.          */
int ach_sgd_update(size_t n, float *w, float *v, float decay_coef, float lr_coef,
                   float momentum, ach_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif
