/*
 * oracle.h -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.
 *
 * A plain-C restatement of the CPU path of onlineaet/aet-cnn for one CNN
 * training step (conv fwd/dgrad/wgrad via im2col+GEMM, batch-norm in training
 * mode, leaky/relu/linear activations, max and global-average pooling with
 * int32 argmax, softmax + cross-entropy, dropout and the SGD momentum/decay
 * update).  Every function cites the reference file:line it follows; paths are
 * relative to /root/reference/src/com/ai/dnn/.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker / CPU baseline.  The HIP product
 * path never calls into it.
 *
 * Parity pinning: every function here is checked in tests/test_oracle.py
 * against closed forms, brute force in double, adjoint identities or exact
 * index maps on tiny shapes (the reference ships no golden vectors).
 */
#ifndef AETCNN_ORACLE_H
#define AETCNN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Activation ids follow the order of the reference's ActivationType enum
 * (Activation.h: LOGISTIC, RELU, RELIE, LINEAR, RAMP, TANH, PLSE, LEAKY, ...);
 * only the three used by the benchmark configs are implemented. */
enum { OR_LOGISTIC = 0, OR_RELU = 1, OR_LINEAR = 3, OR_LEAKY = 7 };

/* ---- runtime knobs ------------------------------------------------------ */
/* 0 = reference-faithful (GEMM single-threaded, Gemm.c:133 pragma commented
 *     out); 1 = oracle-parallel (row-parallel GEMM, same per-element order). */
void or_set_gemm_parallel(int on);
int  or_get_gemm_parallel(void);
int  or_max_threads(void);

/* ---- GEMM (Gemm.c:53-144) ----------------------------------------------- */
void or_gemm(int TA, int TB, int M, int N, int K, float ALPHA,
             const float *A, int lda, const float *B, int ldb,
             float BETA, float *C, int ldc);

/* ---- im2col / col2im, Caffe "ext" variants (Im2Col.c:65-103, 155-192) --- */
void or_im2col(const float *im, int channels, int height, int width,
               int kh, int kw, int ph, int pw, int sh, int sw, int dh, int dw,
               float *col);
void or_col2im(const float *col, int channels, int height, int width,
               int kh, int kw, int ph, int pw, int sh, int sw, int dh, int dw,
               float *im);

/* ---- convolution GEMM parts of ConvolutionalLayer (groups=1, dilation=1) - */
typedef struct {
    int batch, c, h, w;      /* input  [batch][c][h][w]   */
    int n, size, stride, pad;/* filters, kernel, stride (= stride_x), padding */
    int stride_y;            /* height stride; 0: the same as stride       */
} or_conv_shape;
int  or_conv_out_h(const or_conv_shape *s);
int  or_conv_out_w(const or_conv_shape *s);
size_t or_conv_workspace_floats(const or_conv_shape *s);
/* out = 0; per image out_i += W * col(in_i)     (ConvolutionalLayer.c:689,716-803) */
void or_conv_forward(const or_conv_shape *s, const float *in, const float *w,
                     float *out, float *workspace);
/* per image: dW += delta_i * col(in_i)^T; if dx: ws = W^T delta_i, col2im -> dx_i
 *                                                 (ConvolutionalLayer.c:906-947) */
void or_conv_backward(const or_conv_shape *s, const float *in, const float *delta,
                      const float *w, float *dw, float *dx, float *workspace);

/* ---- bias (IOData.c:43-55, BiasData.c:40-57) ----------------------------- */
void or_add_bias(float *out, const float *biases, int batch, int n, int spatial);
void or_bias_grad(float *bias_updates, const float *delta, int batch, int n, int spatial);

/* ---- batch-norm, training mode ------------------------------------------ */
/* NormData.calcVarianceAndMean (NormData.c:141-186): unbiased sum-of-squares */
void or_bn_mean_var(const float *out, int batch, int c, int spatial,
                    float *mean, float *variance);
/* NormData.scalAxpyRollMeanAndRollVariance (NormData.c:224-229): .9/.1     */
void or_bn_roll(int c, const float *mean, const float *variance,
                float *rolling_mean, float *rolling_variance);
/* NormData.normalize (NormData.c:244-282); returns nonzero on NaN (the
 * reference prints and exit(0)s there).                                     */
int  or_bn_normalize(float *out, int batch, int c, int spatial,
                     const float *mean, const float *variance,
                     const float *scales, const float *biases,
                     float *x, float *x_norm);
/* backwardNormCPU (NLayer.c:246-278): dgamma += sum(delta*x_norm); delta *=
 * gamma; mean_delta; variance_delta; delta <- normalize_delta.  No beta grad. */
void or_bn_backward(float *delta, int batch, int c, int spatial,
                    const float *x, const float *x_norm,
                    const float *mean, const float *variance,
                    const float *scales, float *scale_updates,
                    float *mean_delta, float *variance_delta);
/* NormData.normalizeByRoll (NormData.c:291-326): inference-mode BN          */
void or_bn_normalize_roll(float *out, int batch, int c, int spatial,
                          const float *rolling_mean, const float *rolling_variance,
                          const float *scales, const float *biases);

/* ConvolutionalLayer.fuseConvBatchnorm (ConvolutionalLayer.c:983-1003):
 * weights [filters][fsize] and biases [filters] absorb the inference BN
 * (eps 1e-5 under the square root, double arithmetic, one float rounding) */
void or_conv_bn_fold(int filters, int fsize, float *weights, float *biases,
                     const float *scales, const float *rolling_mean,
                     const float *rolling_variance);

/* ---- activations (Activation.h:41-113, Activation.c:160-239) ------------ */
void or_activate(float *x, int n, int act);
void or_gradient(const float *y, int n, int act, float *delta);

/* ---- max-pool (MaxPoolLayer.c:12-55, 237-272, 318-331) ------------------- */
int  or_maxpool_out(int in, int size, int stride, int padding);
void or_maxpool_forward(const float *in, int batch, int c, int h, int w,
                        int size, int stride, int padding,
                        float *out, int *indexes);
/* the same scan with a width stride stride_x and a height stride stride_y
 * (out w = (w + padding - size)/stride_x + 1, h likewise with stride_y)    */
void or_maxpool_forward_xy(const float *in, int batch, int c, int h, int w, int size,
                           int stride_x, int stride_y, int padding, float *out, int *indexes);
void or_maxpool_backward(const float *delta_out, const int *indexes, int n_out,
                         float *delta_in);

/* ---- global average pool (AvgPoolLayer.c:29-46, 73-88) ------------------- */
void or_avgpool_forward(const float *in, int batch, int c, int spatial, float *out);
void or_avgpool_backward(const float *delta_out, int batch, int c, int spatial,
                         float *delta_in);

/* ---- softmax + cross-entropy (SoftMaxLayer.c:47-119, 291-323) ------------ */
/* returns cost = sum(error) (NData.sum, NData.c:321-328)                   */
float or_softmax_xent_forward(const float *in, int batch, int inputs, int groups,
                              float temperature, const float *truth,
                              float *output, float *delta, float *error);
void or_softmax_backward(const float *delta, int n, float *delta_prev);

/* ---- dropout (DropoutLayer.c:55-86) with a counter-based uniform ---------- */
/* r = u(seed, iter, layer, i) replaces the reference's sequential rand()     */
float or_dropout_uniform(uint64_t seed, uint32_t iter, uint32_t layer, uint32_t i);
void or_dropout_forward(float *x, int n, float probability,
                        uint64_t seed, uint32_t iter, uint32_t layer);
void or_dropout_backward(float *delta, int n, float probability,
                         uint64_t seed, uint32_t iter, uint32_t layer);

/* ---- SGD update (ConvolutionalLayer.c:959-980, WeightData.c:45-78,
 *      BiasData.c:79-94, ScaleData.c:48-73) -------------------------------- */
void or_conv_update(int n_weights, float *weights, float *weight_updates,
                    int n, float *biases, float *bias_updates,
                    float *scales, float *scale_updates,
                    int batch, float learning_rate, float momentum, float decay);

/* ---- weight init (WeightData.c:153-166, DnnUtils.c:196-209) ---------------
 * randUniform(-1,1) over glibc rand(): seeded with srand(seed).             */
void or_rand_seed(unsigned seed);
float or_rand_uniform(float min, float max);

/* ---- learning-rate policy (NNetwork.c:215-246; ids in the order of the
 *      LearningRatePolicy enum, NNetwork.h:29-31) --------------------------- */
enum { OR_POLICY_CONSTANT = 0, OR_POLICY_STEP = 1, OR_POLICY_EXP = 2, OR_POLICY_POLY = 3,
       OR_POLICY_STEPS = 4, OR_POLICY_SIG = 5, OR_POLICY_RANDOM = 6 };
/* getCurrentRate at batch_num = seen / (batch * subdivisions)              */
float or_lr_rate(int policy, float learning_rate, uint64_t batch_num, int burn_in, float power,
                 float gamma, float scale, int step, int max_batches, int num_steps,
                 const int *steps, const float *scales);

/* ---- whole network (NNetwork.c:382-396, 627-680, 740-805) ------------------ */
typedef struct or_net or_net;
or_net *or_net_create(int batch, int h, int w, int c);
/* layer constructors return the layer index, or -1 on error                 */
int  or_net_add_conv(or_net *net, int filters, int size, int stride, int pad,
                     int activation, int batch_normalize);
/* fully connected: previous output flattened to c*h*w, then a 1x1 conv   */
int  or_net_add_connected(or_net *net, int outputs, int activation, int batch_normalize);
int  or_net_add_maxpool(or_net *net, int size, int stride, int padding);
/* separate width / height strides (createConvolutional / createMaxPool,
 * NetworkFactory.c:83-90, 545-546: the layer's stride is stride_x)          */
int  or_net_add_conv_xy(or_net *net, int filters, int size, int stride_x, int stride_y, int pad,
                        int activation, int batch_normalize);
int  or_net_add_maxpool_xy(or_net *net, int size, int stride_x, int stride_y, int padding);
int  or_net_add_avgpool(or_net *net);
int  or_net_add_dropout(or_net *net, float probability);
int  or_net_add_softmax(or_net *net, int groups, float temperature);
void or_net_set_hyper(or_net *net, float learning_rate, float momentum, float decay);
void or_net_set_dropout_seed(or_net *net, uint64_t seed);
/* parseNetOption's policy keys (NetworkFactory.c:768-823); steps/scales
 * are copied                                                              */
void or_net_set_policy(or_net *net, int policy, int burn_in, float power, float gamma,
                       float scale, int step, int max_batches, int num_steps, const int *steps,
                       const float *scales);
/* minibatches per update (NNetwork.h:35); batch given to or_net_create is
 * the minibatch                                                           */
void or_net_set_subdivisions(or_net *net, int subdivisions);
/* the rate the next update uses: or_lr_rate at seen/(batch*subdivisions)   */
float or_net_rate(or_net *net);
uint64_t or_net_seen(const or_net *net);
int  or_net_iteration(const or_net *net);
/* NLayer options stopbackward / onlyforward / learning_rate_scale
 * (NLayer.h:115-121); set before or_net_finalize, which freezes the layers
 * below the last stopbackward layer (NetworkFactory.c:981-991)           */
void or_net_set_layer_options(or_net *net, int layer, int stopbackward, int onlyforward,
                              float learning_rate_scale);
int  or_net_finalize(or_net *net);   /* allocates workspace */
void or_net_free(or_net *net);
/* one minibatch on host buffers: input [batch][c][h][w], truth
 * [batch][classes]; forward + backward, then the update after every
 * subdivisions-th minibatch.  Returns that minibatch's sum(cost)/batch.     */
float or_net_train(or_net *net, const float *input, const float *truth);
/* NNetwork.train(input, truth): seen += batch, forward + backward only      */
float or_net_forward_backward(or_net *net, const float *input, const float *truth);
void or_net_update(or_net *net);
/* NNetwork.predict (NNetwork.c:411-422): inference forward (BN with rolling
 * statistics, dropout off, no truth); output = last layer's output          */
void or_net_predict(or_net *net, const float *input, float *output);
/* NNetwork.fuseConvBatchnorm (NNetwork.c:272-288): fold every BN conv layer
 * (or_conv_bn_fold) and clear its batch_normalize flag                     */
void or_net_fuse_conv_batchnorm(or_net *net);
/* per-layer steps with the network's own state (NetworkState of
 * NNetwork.forward/backward): load one batch, then run layer i             */
void or_net_load(or_net *net, const float *input, const float *truth);
void or_net_layer_forward(or_net *net, int i, int train);
void or_net_layer_backward(or_net *net, int i);
float or_net_cost(or_net *net);

/* introspection for tests */
int  or_net_n_layers(const or_net *net);
/* which: 0 output,1 delta,2 weights,3 weight_updates,4 biases,5 bias_updates,
 *        6 scales,7 scale_updates,8 rolling_mean,9 rolling_variance,10 mean,
 *        11 variance,12 x,13 x_norm,14 indexes(int), 15 loss(per element) */
void *or_net_buffer(or_net *net, int layer, int which, size_t *count);
/* layer meta: type(0 conv,1 maxpool,2 avgpool,3 dropout,4 softmax), out c/h/w */
void or_net_layer_info(const or_net *net, int layer, int *info8);

#ifdef __cplusplus
}
#endif
#endif
