/*
 * network.c -- the reference's network runtime and layer objects as plain C,
 * driving the HIP kernels through aetcnn_ops.h only.  Paths are relative to
 * /root/reference/src/com/ai/dnn/.
 *
 * Memory: every per-layer tensor lives in one device arena; all conv weights
 * (and their momentum buffers) are contiguous so the SGD update of the whole
 * network is two launches (decayed weights; biases + scales without decay)
 * instead of the reference GPU path's five launches per layer
 * (mtcs/MtcsConvLayer.c:618-630).
 */
#include "aetcnn_net.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define AN_CHECK(expr)                \
    do {                              \
        int rc_ = (expr);             \
        if (rc_ != ACH_OK) return rc_; \
    } while (0)

struct an_network {
    int batch, h, w, c, inputs;
    int n, cap;
    an_layer **layers;
    float learning_rate, momentum, decay;
    uint64_t dropout_seed;
    int cur_iteration;
    uint64_t seen;
    /* minibatches per update (NNetwork.h:35); batch is the minibatch       */
    int subdivisions;
    /* index seen/batch of the current minibatch, taken before seen += batch:
     * the step index of its dropout masks                                  */
    uint32_t dropout_step;
    /* learning-rate policy (NNetwork.h:29-31,39,45-51)                     */
    int policy, burn_in, step, max_batches, num_steps;
    float power, gamma, scale;
    int *steps;
    float *scales;
    int finalized;
    ach_stream_t stream;
    /* device memory */
    void *arena;
    size_t arena_bytes;
    float *workspace;
    size_t workspace_bytes;
    float *input, *truth;
    int classes;
    float *wflat, *vflat;          /* all conv weights / weight_updates     */
    size_t nweights_total;
    float *bflat, *bvflat;         /* biases (+scales) / their updates       */
    size_t nbias_total;
    float *wtflat, *wftflat;       /* k-major / flipped k-major filters    */
    /* weight gradients run on a second stream, overlapping the input-gradient
     * chain: its own workspace, one "delta ready" event per layer and one
     * event that joins it back before the update                           */
    ach_stream_t wstream;
    float *wgrad_ws;
    size_t wgrad_ws_bytes;
    void **ev_ready;
    void **ev_dgrad;               /* per layer: its input gradient enqueued */
    /* set by an_train_step around a step that updates: each conv layer's
     * SGD update is enqueued right after its gradients (early_rate)       */
    int early_update;
    float early_rate;
    /* set by an_backward (the whole loop, not the per-layer entry point):
     * a max-pool applies the previous conv layer's activation gradient to
     * the delta it writes, and that layer skips its own pass             */
    int in_chain;
    void *ev_joined;
    ach_filter_job *jobs;          /* one per conv layer                    */
    int njobs;
    float *zero_region;            /* deltas that need zeroing per forward */
    size_t zero_floats;
    /* host copies of initial parameters until finalize */
    float **init_w;
    /* some layer sets stopbackward / onlyforward / a learning-rate scale, or
     * is frozen (train = 0): updates then run layer by layer after the
     * backward loop instead of the flat or early forms                     */
    int layer_opts;
    /* the reference's NaN checks (NormData.c:273-276, ScaleData.c:51-54,
     * 67-70) as one scan per step over every batch-norm layer's mean,
     * variance, scales and scale updates (device table of spans); the flag
     * keeps the smallest tag, layer * 4 + (0 mean, 1 variance, 2 scales,
     * 3 scale updates), of an array holding a NaN, INT32_MAX while clean   */
    ach_nan_span *d_nan_spans;
    int n_nan_spans;
    int32_t *d_nan_flag;
};

/* ---- randUniform over glibc rand() (DnnUtils.c:196-209) ------------------- */
void an_rand_seed(unsigned seed) { srand(seed); }

static float rand_uniform(float min, float max)
{
    if (max < min) {
        float s = min;
        min = max;
        max = s;
    }
    return ((float)rand() / RAND_MAX * (max - min)) + min;
}

an_network *an_network_create(int batch, int h, int w, int c)
{
    if (batch <= 0 || h <= 0 || w <= 0 || c <= 0) return NULL;
    an_network *net = (an_network *)calloc(1, sizeof(an_network));
    if (!net) return NULL;
    net->batch = batch;
    net->h = h;
    net->w = w;
    net->c = c;
    net->inputs = h * w * c;
    /* parseNetOption defaults (NetworkFactory.c:677-685) */
    net->learning_rate = .001f;
    net->momentum = .9f;
    net->decay = .0001f;
    net->dropout_seed = 0x5eed;
    net->subdivisions = 1;
    /* policy defaults (NetworkFactory.c:763-773,817) */
    net->policy = AN_POLICY_CONSTANT;
    net->power = 4;
    net->gamma = 1;
    net->scale = 1;
    net->step = 1;
    return net;
}

static an_layer *push_layer(an_network *net)
{
    if (net->finalized) return NULL;
    if (net->n == net->cap) {
        int cap = net->cap ? 2 * net->cap : 16;
        an_layer **nl = (an_layer **)realloc(net->layers, sizeof(an_layer *) * cap);
        float **ni = (float **)realloc(net->init_w, sizeof(float *) * cap);
        if (!nl || !ni) return NULL;
        net->layers = nl;
        net->init_w = ni;
        net->cap = cap;
    }
    an_layer *l = (an_layer *)calloc(1, sizeof(an_layer));
    if (!l) return NULL;
    l->index = net->n;
    l->batch = net->batch;
    if (net->n == 0) {
        l->h = net->h;
        l->w = net->w;
        l->c = net->c;
    } else {
        an_layer *p = net->layers[net->n - 1];
        l->h = p->out_h;
        l->w = p->out_w;
        l->c = p->out_c;
    }
    l->inputs = l->h * l->w * l->c;
    l->train = 1;
    l->learning_rate_scale = 1.f;
    net->layers[net->n] = l;
    net->init_w[net->n] = NULL;
    return l;
}

/* ======================================================================== */
/* Convolutional layer: ConvolutionalLayer.c:684-854 (forward), :863-948
 * (backward), :959-980 (update).                                          */
static ach_conv_desc conv_desc(const an_layer *l)
{
    ach_conv_desc d;
    d.batch = l->batch;
    d.c = l->c;
    d.h = l->h;
    d.w = l->w;
    d.n = l->n;
    d.size = l->size;
    d.stride = l->stride_x;
    d.pad = l->pad;
    d.stride_y = l->stride_y;
    return d;
}

static int fusable(int act) { return act == ACH_LEAKY || act == ACH_RELU || act == ACH_LINEAR; }

static int conv_forward(an_network *net, an_layer *l, an_state st)
{
    ach_conv_desc d = conv_desc(l);
    const int spatial = l->out_h * l->out_w;
    ach_stream_t s = net->stream;
    if (l->batch_normalize) {
        /* conv output goes straight into NormData.x; BN writes output */
        AN_CHECK(ach_conv_fwd_prepared(&d, st.input, l->weights_kmajor, l->x, st.workspace,
                                       st.workspace_bytes, s));
        const int act = fusable(l->activation) ? l->activation : ACH_LINEAR;
        if (st.train)
            AN_CHECK(ach_bn_train_fwd_from_x(l->x, l->output, l->batch, l->n, spatial,
                                             l->scales, l->biases, l->mean, l->variance,
                                             l->rolling_mean, l->rolling_variance, act,
                                             st.workspace, st.workspace_bytes, s));
        else /* forwardNormCPU test branch: normalizeByRoll (NormData.c:291-326) */
            AN_CHECK(ach_bn_infer(l->x, l->output, l->batch, l->n, spatial, l->scales,
                                  l->biases, l->rolling_mean, l->rolling_variance, act, s));
        if (!fusable(l->activation))
            AN_CHECK(ach_activate(l->output, (size_t)l->batch * l->outputs, l->activation, s));
        return ACH_OK;
    }
    /* conv + addBias + activate in one pass (the GEMM epilogue) */
    if (fusable(l->activation) || l->activation == ACH_LOGISTIC)
        return ach_conv_fwd_bias_act_prepared(&d, st.input, l->weights_kmajor, l->biases,
                                              l->activation, l->output, st.workspace,
                                              st.workspace_bytes, s);
    AN_CHECK(ach_conv_fwd_prepared(&d, st.input, l->weights_kmajor, l->output, st.workspace,
                                   st.workspace_bytes, s));
    AN_CHECK(ach_add_bias(l->output, l->biases, l->batch, l->n, spatial, s));
    return ach_activate(l->output, (size_t)l->batch * l->outputs, l->activation, s);
}

/* A dropout layer right above l that shares l's output (masked in place by
 * its forward) but whose backward is skipped (onlyforward): l's delta is
 * then not masked, and the reference takes l's activation gradient from the
 * masked output (Activation.gradientArray on outputData, f'(0) where a unit
 * was dropped).  The BN passes derive the gradient's sign from the
 * recomputed pre-activation instead, which equals f'(y) only where the
 * output was not masked or its delta is zero.                             */
static int output_masked_unreverted(const an_network *net, const an_layer *l)
{
    if (l->index + 1 >= net->n) return 0;
    const an_layer *d = net->layers[l->index + 1];
    return d->type == AN_DROPOUT && d->shares_prev && d->onlyforward;
}

/* ConvolutionalLayer.backward's input gradient into state.delta
 * (ConvolutionalLayer.c:931-945): the GEMM path for stride 1, the
 * reference's per-image GEMM + col2im otherwise                          */
static int conv_input_gradient(const an_layer *l, const ach_conv_desc *d, an_state st,
                               ach_stream_t s)
{
    return l->stride_x == 1 && l->stride_y == 1
               ? ach_conv_bwd_data_prepared(d, l->delta, l->weights, l->weights_flipped, st.delta,
                                            st.workspace, st.workspace_bytes, s)
               : ach_conv_bwd_data(d, l->delta, l->weights, st.delta, st.workspace,
                                   st.workspace_bytes, s);
}

static int conv_backward(an_network *net, an_layer *l, an_state st)
{
    ach_conv_desc d = conv_desc(l);
    const int spatial = l->out_h * l->out_w;
    ach_stream_t s = net->stream;
    const size_t nout = (size_t)l->batch * l->outputs;
    if (l->batch_normalize) {
        int act = ACH_LINEAR;
        if ((l->activation == ACH_LEAKY || l->activation == ACH_RELU) &&
            !output_masked_unreverted(net, l))
            act = l->activation; /* gradient fused into the BN passes */
        else
            AN_CHECK(ach_gradient(l->output, nout, l->activation, l->delta, s));
        AN_CHECK(ach_bn_bwd(l->delta, l->batch, l->n, spatial, l->x, NULL, l->mean,
                            l->variance, l->scales, l->biases, l->scale_updates,
                            l->mean_delta, l->variance_delta, act, st.workspace,
                            st.workspace_bytes, s));
    } else if (l->grad_applied) {
        l->grad_applied = 0; /* the max-pool above applied f'(y) already */
    } else if (l->bias_planes && l->activation != ACH_LINEAR) {
        /* the gradient pass also takes the bias gradient's plane sums */
        AN_CHECK(ach_gradient_planes(l->output, l->batch, l->n, spatial, l->activation, l->delta,
                                     l->bias_planes, s));
        l->planes_ready = 1;
    } else {
        AN_CHECK(ach_gradient(l->output, nout, l->activation, l->delta, s));
    }
    /* dbias and dW on the weight-gradient stream once delta is final, while
     * the input gradient continues on the main stream.  A layer without an
     * input gradient (the first) computes them on the main stream, which has
     * nothing else left to do, so they overlap the weight gradients still
     * queued on the other stream instead of waiting behind them.          */
    ach_stream_t gs = s;
    float *gws = st.workspace;
    size_t gws_bytes = st.workspace_bytes;
    if (st.delta) {
        AN_CHECK(ach_event_record(net->ev_ready[l->index], s));
        AN_CHECK(ach_stream_wait_event(net->wstream, net->ev_ready[l->index]));
        gs = net->wstream;
        gws = net->wgrad_ws;
        gws_bytes = net->wgrad_ws_bytes;
    }
    if (!l->batch_normalize && l->planes_ready) {
        l->planes_ready = 0;
        AN_CHECK(ach_bias_grad_planes(l->bias_updates, l->bias_planes, l->batch, l->n, gs));
    } else if (!l->batch_normalize) {
        AN_CHECK(ach_bias_grad(l->bias_updates, l->delta, l->batch, l->n, spatial, gws,
                               gws_bytes, gs));
    }
    const int ub = net->batch * net->subdivisions;
    if (net->early_update) {
        /* The layer's SGD update (ConvolutionalLayer.update, the per-layer
         * step of NNetwork.updateCPU) as soon as nothing else reads its
         * parameters: the weights' step rides on the pass that finishes
         * the weight gradient (ach_conv_bwd_filter_sgd), after the input
         * gradient when that reads W (otherwise it reads the flipped copy
         * made at the forward); biases and scales follow on the same
         * stream.  The same arithmetic as an_update; it overlaps the
         * backward of the layers below instead of ending the step
         * (AlexNet's FC weights are 94% of its parameters).               */
        const int reads_w = st.delta && ach_conv_bwd_data_reads_w(&d);
        if (reads_w) {
            AN_CHECK(conv_input_gradient(l, &d, st, s));
            AN_CHECK(ach_event_record(net->ev_dgrad[l->index], s));
            AN_CHECK(ach_stream_wait_event(gs, net->ev_dgrad[l->index]));
        }
        AN_CHECK(ach_conv_bwd_filter_sgd(&d, st.input, l->delta, l->weights, l->weight_updates,
                                         -net->decay * ub, net->early_rate / ub, net->momentum,
                                         gws, gws_bytes, gs));
        if (st.delta && !reads_w) AN_CHECK(conv_input_gradient(l, &d, st, s));
        return ach_conv_update(0, NULL, NULL, (size_t)l->n, l->biases, l->bias_updates,
                               l->scales, l->scale_updates, ub, net->early_rate, net->momentum,
                               net->decay, gs);
    }
    AN_CHECK(ach_conv_bwd_filter(&d, st.input, l->delta, l->weight_updates, gws, gws_bytes,
                                 gs));
    if (st.delta) AN_CHECK(conv_input_gradient(l, &d, st, s));
    return ACH_OK;
}

/* per-layer update for callers that drive layers one by one; an_update
 * uses the flat buffers instead (same arithmetic, fewer launches).        */
static int conv_update(an_network *net, an_layer *l, int batch, float lr, float momentum,
                       float decay)
{
    return ach_conv_update((size_t)l->nweights, l->weights, l->weight_updates, (size_t)l->n,
                           l->biases, l->bias_updates, l->scales, l->scale_updates, batch, lr,
                           momentum, decay, net->stream);
}

/* flatten != 0: the layer reads the previous output [batch][c][h][w] as
 * [batch][c*h*w][1][1] (the same memory), for an_add_connected */
static int add_conv(an_network *net, int filters, int size, int stride_x, int stride_y, int pad,
                    int activation, int batch_normalize, int flatten)
{
    if (!net || filters <= 0 || size <= 0 || stride_x <= 0 || stride_y <= 0 || pad < 0)
        return ACH_EINVAL;
    if (activation != ACH_LEAKY && activation != ACH_RELU && activation != ACH_LINEAR &&
        activation != ACH_LOGISTIC)
        return ACH_EUNSUPPORTED;
    an_layer *l = push_layer(net);
    if (!l) return ACH_EINVAL;
    if (flatten) {
        l->c = l->c * l->h * l->w;
        l->h = l->w = 1;
        l->connected = 1;
    }
    l->type = AN_CONVOLUTIONAL;
    l->n = filters;
    l->size = size;
    l->stride = l->stride_x = stride_x;
    l->stride_y = stride_y;
    l->pad = pad;
    l->activation = activation;
    l->batch_normalize = batch_normalize ? 1 : 0;
    l->out_h = (l->h + 2 * pad - size) / stride_y + 1;
    l->out_w = (l->w + 2 * pad - size) / stride_x + 1;
    l->out_c = filters;
    if (l->h + 2 * pad < size || l->w + 2 * pad < size || l->out_h <= 0 || l->out_w <= 0) {
        free(l);
        return ACH_EINVAL;
    }
    l->outputs = l->out_h * l->out_w * l->out_c;
    l->nweights = l->c * filters * size * size;
    l->forward = conv_forward;
    l->backward = conv_backward;
    l->update = conv_update;
    /* ConvKernel.initData (WeightData.c:153-166), in construction order */
    float *w = (float *)malloc(sizeof(float) * l->nweights);
    if (!w) {
        free(l);
        return ACH_EINVAL;
    }
    const float scale = sqrt(2. / (size * size * l->c));
    for (int i = 0; i < l->nweights; ++i) w[i] = scale * rand_uniform(-1, 1);
    net->init_w[net->n] = w;
    return net->n++;
}

int an_add_convolutional(an_network *net, int filters, int size, int stride, int pad,
                         int activation, int batch_normalize)
{
    return add_conv(net, filters, size, stride, stride, pad, activation, batch_normalize, 0);
}

int an_add_convolutional_xy(an_network *net, int filters, int size, int stride_x, int stride_y,
                            int pad, int activation, int batch_normalize)
{
    return add_conv(net, filters, size, stride_x, stride_y, pad, activation, batch_normalize, 0);
}

/* A fully connected layer: the previous output flattened to c*h*w features
 * per image, y = act(W x + b) (or BN) with W [outputs][inputs]; it runs as a
 * 1x1 convolution of the flattened input, so the GEMM kernels take their
 * fully connected path.  Init sqrt(2/inputs)*randUniform(-1,1), which is
 * the convolution's rule with k = 1. */
int an_add_connected(an_network *net, int outputs, int activation, int batch_normalize)
{
    return add_conv(net, outputs, 1, 1, 1, 0, activation, batch_normalize, 1);
}

/* ======================================================================== */
/* Max-pool: MaxPoolLayer.c:237-272 / :318-331, defaults from createMaxPool
 * (NetworkFactory.c:543-570: padding = size-1 unless given).              */
/* the conv layer whose delta a max-pool's input gradient is, when the pool
 * applies that layer's activation gradient (whole backward loop only)    */
static an_layer *pool_act_target(an_network *net, const an_layer *l, const float *delta)
{
    an_layer *p = l->index > 0 ? net->layers[l->index - 1] : NULL;
    if (net->in_chain && p && p->type == AN_CONVOLUTIONAL && !p->batch_normalize &&
        p->delta == delta && p->activation != ACH_LINEAR)
        return p;
    return NULL;
}

static int maxpool_forward(an_network *net, an_layer *l, an_state st)
{
    return ach_maxpool_fwd_xy(st.input, l->batch, l->c, l->h, l->w, l->size, l->stride_x,
                              l->stride_y, l->pad, l->output, l->indexes, net->stream);
}

static int maxpool_backward(an_network *net, an_layer *l, an_state st)
{
    if (!st.delta) return ACH_OK;
    /* unequal strides: the general gather, and the layer below applies its
     * own activation gradient */
    if (l->stride_x != l->stride_y)
        return ach_maxpool_bwd_xy(l->delta, l->indexes, l->batch, l->c, l->h, l->w, l->size,
                                  l->stride_x, l->stride_y, l->pad, st.delta, 0, net->stream);
    /* the only contribution to the previous delta, which the reference
     * zeroes in forward: write the sums instead of adding to zeros.  In the
     * whole backward loop, when that delta is a plain conv layer's own (no
     * BN, which fuses its gradient itself), the layer's activation gradient
     * is applied here and the conv layer's backward skips it.              */
    an_layer *p = pool_act_target(net, l, st.delta);
    const int out_kept = l->index + 1 >= net->n || !net->layers[l->index + 1]->shares_prev;
    if (p && out_kept && (p->activation == ACH_RELU || p->activation == ACH_LEAKY)) {
        /* ... from the pool's own output, which a following layer has not
         * masked in place: the gradient at each argmax pixel, read from the
         * pooled tensor instead of the conv output                          */
        const int rc = ach_maxpool_bwd_act_pooled(l->delta, l->indexes, l->batch, l->c, l->h,
                                                  l->w, l->size, l->stride, l->pad, st.delta,
                                                  l->output, p->activation, p->bias_planes,
                                                  net->stream);
        if (rc == ACH_OK) {
            p->grad_applied = 1;
            p->planes_ready = p->bias_planes != NULL;
            return ACH_OK;
        }
        if (rc != ACH_EUNSUPPORTED) return rc;
    }
    if (p && p->bias_planes) {
        /* ... and takes that layer's bias-gradient plane sums as it writes */
        const int rc = ach_maxpool_bwd_act_planes(l->delta, l->indexes, l->batch, l->c, l->h,
                                                  l->w, l->size, l->stride, l->pad, st.delta,
                                                  p->output, p->activation, p->bias_planes,
                                                  net->stream);
        if (rc == ACH_OK) {
            p->grad_applied = 1;
            p->planes_ready = 1;
            return ACH_OK;
        }
        if (rc != ACH_EUNSUPPORTED) return rc;
    }
    if (p) {
        AN_CHECK(ach_maxpool_bwd_act(l->delta, l->indexes, l->batch, l->c, l->h, l->w, l->size,
                                     l->stride, l->pad, st.delta, 0, p->output, p->activation,
                                     net->stream));
        p->grad_applied = 1;
        return ACH_OK;
    }
    return ach_maxpool_bwd(l->delta, l->indexes, l->batch, l->c, l->h, l->w, l->size, l->stride,
                           l->pad, st.delta, 0, net->stream);
}

int an_add_maxpool(an_network *net, int size, int stride, int padding)
{
    return an_add_maxpool_xy(net, size, stride, stride, padding);
}

int an_add_maxpool_xy(an_network *net, int size, int stride_x, int stride_y, int padding)
{
    if (!net || size <= 0 || stride_x <= 0 || stride_y <= 0 || padding < 0) return ACH_EINVAL;
    an_layer *l = push_layer(net);
    if (!l) return ACH_EINVAL;
    l->type = AN_MAXPOOL;
    l->size = size;
    l->stride = l->stride_x = stride_x;
    l->stride_y = stride_y;
    l->pad = padding;
    l->out_h = ach_maxpool_out(l->h, size, stride_y, padding);
    l->out_w = ach_maxpool_out(l->w, size, stride_x, padding);
    l->out_c = l->c;
    if (l->out_h <= 0 || l->out_w <= 0) {
        free(l);
        return ACH_EINVAL;
    }
    l->outputs = l->out_h * l->out_w * l->out_c;
    l->forward = maxpool_forward;
    l->backward = maxpool_backward;
    return net->n++;
}

/* ======================================================================== */
/* Global average pool: AvgPoolLayer.c:17-88.                               */
static int avgpool_forward(an_network *net, an_layer *l, an_state st)
{
    return ach_avgpool_fwd(st.input, l->batch, l->c, l->h * l->w, l->output, net->stream);
}

static int avgpool_backward(an_network *net, an_layer *l, an_state st)
{
    if (!st.delta) return ACH_OK;
    return ach_avgpool_bwd(l->delta, l->batch, l->c, l->h * l->w, st.delta, net->stream);
}

int an_add_avgpool(an_network *net)
{
    if (!net) return ACH_EINVAL;
    an_layer *l = push_layer(net);
    if (!l) return ACH_EINVAL;
    l->type = AN_AVGPOOL;
    l->out_h = l->out_w = 1;
    l->out_c = l->c;
    l->outputs = l->c;
    l->forward = avgpool_forward;
    l->backward = avgpool_backward;
    return net->n++;
}

/* ======================================================================== */
/* Dropout: DropoutLayer.c:55-86; shares the previous layer's output and
 * delta (NetworkFactory.c:644-650).                                        */
static int dropout_forward(an_network *net, an_layer *l, an_state st)
{
    if (!st.train) return ACH_OK;
    const size_t n = (size_t)l->batch * l->inputs;
    return ach_dropout_fwd((float *)st.input, n, l->probability, net->dropout_seed,
                           net->dropout_step, (uint32_t)l->index, net->stream);
}

static int dropout_backward(an_network *net, an_layer *l, an_state st)
{
    if (!st.delta) return ACH_OK;
    const size_t n = (size_t)l->batch * l->inputs;
    return ach_dropout_bwd(st.delta, n, l->probability, net->dropout_seed,
                           net->dropout_step, (uint32_t)l->index, net->stream);
}

int an_add_dropout(an_network *net, float probability)
{
    if (!net || net->n == 0 || !(probability >= 0.f && probability < 1.f)) return ACH_EINVAL;
    an_layer *l = push_layer(net);
    if (!l) return ACH_EINVAL;
    l->type = AN_DROPOUT;
    l->probability = probability;
    l->out_h = l->h;
    l->out_w = l->w;
    l->out_c = l->c;
    l->outputs = l->inputs;
    l->shares_prev = 1;
    l->forward = dropout_forward;
    l->backward = dropout_backward;
    return net->n++;
}

/* ======================================================================== */
/* Softmax + cross-entropy: SoftMaxLayer.c:99-119, :291-316.                */
static int softmax_forward(an_network *net, an_layer *l, an_state st)
{
    return ach_softmax_xent(st.input, l->batch, l->inputs, l->groups, l->temperature,
                            st.truth, l->output, l->delta, l->loss, l->cost, st.workspace,
                            st.workspace_bytes, net->stream);
}

static int softmax_backward(an_network *net, an_layer *l, an_state st)
{
    if (!st.delta) return ACH_OK;
    return ach_axpy((size_t)l->batch * l->inputs, 1.f, l->delta, st.delta, net->stream);
}

int an_add_softmax(an_network *net, int groups, float temperature)
{
    if (!net || groups <= 0) return ACH_EINVAL;
    an_layer *l = push_layer(net);
    if (!l) return ACH_EINVAL;
    if (l->inputs % groups) {
        free(l);
        return ACH_EINVAL;
    }
    l->type = AN_SOFTMAX;
    l->groups = groups;
    l->temperature = temperature;
    l->out_h = l->h;
    l->out_w = l->w;
    l->out_c = l->c;
    l->outputs = l->inputs;
    l->forward = softmax_forward;
    l->backward = softmax_backward;
    return net->n++;
}

void an_set_hyper(an_network *net, float learning_rate, float momentum, float decay)
{
    net->learning_rate = learning_rate;
    net->momentum = momentum;
    net->decay = decay;
}

void an_set_dropout_seed(an_network *net, uint64_t seed)
{
    net->dropout_seed = seed;
}

int an_set_policy(an_network *net, int policy, int burn_in, float power, float gamma,
                  float scale, int step, int max_batches, int num_steps, const int *steps,
                  const float *scales)
{
    if (!net || policy < AN_POLICY_CONSTANT || policy > AN_POLICY_RANDOM || num_steps < 0 ||
        (num_steps && (!steps || !scales)) || (policy == AN_POLICY_STEPS && !num_steps) ||
        ((policy == AN_POLICY_STEP || policy == AN_POLICY_SIG) && step <= 0) || burn_in < 0)
        return ACH_EINVAL;
    int *st = NULL;
    float *sc = NULL;
    if (num_steps) {
        st = (int *)malloc(sizeof(int) * num_steps);
        sc = (float *)malloc(sizeof(float) * num_steps);
        if (!st || !sc) {
            free(st);
            free(sc);
            return ACH_EINVAL; /* host allocation failed */
        }
        memcpy(st, steps, sizeof(int) * num_steps);
        memcpy(sc, scales, sizeof(float) * num_steps);
    }
    free(net->steps);
    free(net->scales);
    net->steps = st;
    net->scales = sc;
    net->num_steps = num_steps;
    net->policy = policy;
    net->burn_in = burn_in;
    net->power = power;
    net->gamma = gamma;
    net->scale = scale;
    net->step = step;
    net->max_batches = max_batches;
    return ACH_OK;
}

int an_set_subdivisions(an_network *net, int subdivisions)
{
    if (!net || subdivisions < 1) return ACH_EINVAL;
    net->subdivisions = subdivisions;
    return ACH_OK;
}

/* NNetwork.getCurrentRate (NNetwork.c:215-246) with the reference's types:
 * batch_num is size_t (getCurrentBatch, NNetwork.c:154-157), so in the
 * sigmoid policy batch_num - step wraps around below step (the rate is
 * then 0 for gamma > 0), and burn_in and steps[i] compare as size_t.  The
 * random policy draws randUniform(0,1) from rand() (DnnUtils.c:196-209).  */
float an_rate(an_network *net, uint64_t batch_num64)
{
    const size_t batch_num = (size_t)batch_num64;
    const float lr = net->learning_rate;
    if (batch_num < (size_t)net->burn_in)
        return lr * pow((float)batch_num / net->burn_in, net->power);
    switch (net->policy) {
    case AN_POLICY_STEP: return lr * pow(net->scale, batch_num / (size_t)net->step);
    case AN_POLICY_STEPS: {
        float rate = lr;
        for (int i = 0; i < net->num_steps; ++i) {
            if ((size_t)net->steps[i] > batch_num) return rate;
            rate *= net->scales[i];
        }
        return rate;
    }
    case AN_POLICY_EXP: return lr * pow(net->gamma, (int)batch_num);
    case AN_POLICY_POLY: return lr * pow(1 - (float)batch_num / net->max_batches, net->power);
    case AN_POLICY_RANDOM: return lr * pow(rand_uniform(0, 1), net->power);
    case AN_POLICY_SIG:
        return lr * (1. / (1. + exp(net->gamma * (float)(batch_num - (size_t)net->step))));
    default: return lr;
    }
}

/* ======================================================================== */
/* Arena layout and workspace sizing (NetworkFactory.c:999-1005 sizes one
 * shared workspace to the largest layer need).                             */
static size_t al(size_t bytes) { return (bytes + 255) & ~(size_t)255; }

typedef struct {
    char *base;
    size_t off;
    int dry;
} bump;

static void *take(bump *b, size_t bytes)
{
    void *p = b->dry ? NULL : (void *)(b->base + b->off);
    b->off += al(bytes);
    return p;
}

static size_t layer_ws(const an_layer *l, int batch)
{
    size_t ws = 0;
    if (l->type == AN_CONVOLUTIONAL) {
        ach_conv_desc d = conv_desc(l);
        size_t a = ach_conv_fwd_workspace(&d), b = ach_conv_bwd_data_workspace(&d),
               c = ach_conv_bwd_filter_workspace(&d);
        ws = a > b ? a : b;
        ws = ws > c ? ws : c;
        /* the bias-gradient size too for BN layers: an_fuse_conv_batchnorm
         * turns them into plain conv layers that may still be trained */
        size_t n = ach_bias_grad_workspace(batch, l->n, l->out_h * l->out_w);
        ws = ws > n ? ws : n;
        n = l->batch_normalize ? ach_bn_workspace(batch, l->n, l->out_h * l->out_w) : 0;
        ws = ws > n ? ws : n;
    } else if (l->type == AN_SOFTMAX) {
        ws = ach_softmax_workspace(batch, l->groups);
    }
    return ws;
}

/* lay out every device tensor; b->dry only measures */
static void layout(an_network *net, bump *b)
{
    const size_t B = (size_t)net->batch;
    /* 1. deltas that must be zeroed each forward, contiguous */
    size_t zstart = b->off;
    for (int i = 0; i < net->n; ++i) {
        an_layer *l = net->layers[i];
        if (l->shares_prev || !l->zero_delta) continue;
        l->delta = (float *)take(b, sizeof(float) * B * l->outputs);
    }
    net->zero_region = b->dry ? NULL : (float *)(b->base + zstart);
    net->zero_floats = (b->off - zstart) / sizeof(float);
    /* 2. per-layer tensors (flat parameters are carved by an_finalize) */
    for (int i = 0; i < net->n; ++i) {
        an_layer *l = net->layers[i];
        const size_t bo = B * l->outputs;
        if (l->shares_prev) {
            if (!b->dry) {
                l->output = net->layers[i - 1]->output;
                l->delta = net->layers[i - 1]->delta;
            }
            continue;
        }
        l->output = (float *)take(b, sizeof(float) * bo);
        if (!l->zero_delta) l->delta = (float *)take(b, sizeof(float) * bo);
        if (l->type == AN_CONVOLUTIONAL && l->batch_normalize) {
            l->x = (float *)take(b, sizeof(float) * bo);
            l->mean = (float *)take(b, sizeof(float) * l->n);
            l->variance = (float *)take(b, sizeof(float) * l->n);
            l->rolling_mean = (float *)take(b, sizeof(float) * l->n);
            l->rolling_variance = (float *)take(b, sizeof(float) * l->n);
            l->mean_delta = (float *)take(b, sizeof(float) * l->n);
            l->variance_delta = (float *)take(b, sizeof(float) * l->n);
        } else if (l->type == AN_MAXPOOL) {
            l->indexes = (int32_t *)take(b, sizeof(int32_t) * bo);
        } else if (l->type == AN_CONVOLUTIONAL && l->out_h * l->out_w >= 128) {
            l->bias_planes = (double *)take(b, sizeof(double) * B * l->n);
        } else if (l->type == AN_SOFTMAX) {
            l->loss = (float *)take(b, sizeof(float) * bo);
            l->cost = (float *)take(b, sizeof(float) * 4);
        }
    }
    /* 3. input, truth, workspace */
    net->input = (float *)take(b, sizeof(float) * B * net->inputs);
    net->truth = (float *)take(b, sizeof(float) * B * (net->classes > 0 ? net->classes : 1));
    size_t ws = 0;
    for (int i = 0; i < net->n; ++i) {
        size_t w = layer_ws(net->layers[i], net->batch);
        if (w > ws) ws = w;
    }
    net->workspace_bytes = ws;
    net->workspace = (float *)take(b, ws ? ws : 256);
    size_t wws = 0;
    for (int i = 0; i < net->n; ++i) {
        const an_layer *l = net->layers[i];
        if (l->type != AN_CONVOLUTIONAL) continue;
        ach_conv_desc d = conv_desc(l);
        size_t w = ach_conv_bwd_filter_workspace(&d);
        if (w > wws) wws = w;
        w = ach_bias_grad_workspace(l->batch, l->n, l->out_h * l->out_w);
        if (w > wws) wws = w;
    }
    net->wgrad_ws_bytes = wws;
    net->wgrad_ws = (float *)take(b, wws ? wws : 256);
}

int an_set_layer_options(an_network *net, int layer, const an_layer_options *opt)
{
    an_layer *l = an_get_layer(net, layer);
    if (!l || !opt || net->finalized) return ACH_EINVAL;
    if (opt->flipped && l->type != AN_CONVOLUTIONAL) return ACH_EINVAL;
    l->stopbackward = opt->stopbackward; /* raw: only 1 freezes the layers below */
    l->onlyforward = opt->onlyforward ? 1 : 0;
    l->dontload = opt->dontload ? 1 : 0;
    l->dontloadscales = opt->dontloadscales ? 1 : 0;
    l->flipped = opt->flipped ? 1 : 0;
    l->learning_rate_scale = opt->learning_rate_scale;
    return ACH_OK;
}

int an_get_layer_options(const an_network *net, int layer, an_layer_options *opt)
{
    if (!net || layer < 0 || layer >= net->n || !opt) return ACH_EINVAL;
    const an_layer *l = net->layers[layer];
    opt->stopbackward = l->stopbackward;
    opt->onlyforward = l->onlyforward;
    opt->dontload = l->dontload;
    opt->dontloadscales = l->dontloadscales;
    opt->flipped = l->flipped;
    opt->learning_rate_scale = l->learning_rate_scale;
    return ACH_OK;
}

/* the NaN scan's span table and flag (their own small allocation) */
static int setup_nan_scan(an_network *net)
{
    int nbn = 0;
    for (int i = 0; i < net->n; ++i)
        if (net->layers[i]->type == AN_CONVOLUTIONAL && net->layers[i]->batch_normalize) ++nbn;
    if (!nbn) return ACH_OK;
    ach_nan_span *h = (ach_nan_span *)calloc((size_t)nbn * 4, sizeof(ach_nan_span));
    if (!h) return ACH_EINVAL;
    int k = 0;
    for (int i = 0; i < net->n; ++i) {
        const an_layer *l = net->layers[i];
        if (l->type != AN_CONVOLUTIONAL || !l->batch_normalize) continue;
        const float *arr[4] = {l->mean, l->variance, l->scales, l->scale_updates};
        for (int j = 0; j < 4; ++j, ++k) {
            h[k].p = arr[j];
            h[k].n = (uint64_t)l->n;
            h[k].tag = i * 4 + j;
        }
    }
    const size_t tb = (sizeof(ach_nan_span) * (size_t)k + 255) & ~(size_t)255;
    void *mem = NULL;
    int rc = ach_malloc(&mem, tb + 256);
    const int32_t clean = INT32_MAX;
    if (!rc) rc = ach_memcpy_h2d(mem, h, sizeof(ach_nan_span) * (size_t)k, net->stream);
    if (!rc) rc = ach_memcpy_h2d((char *)mem + tb, &clean, sizeof(clean), net->stream);
    if (!rc) rc = ach_stream_sync(net->stream);
    free(h);
    if (rc) {
        ach_free(mem);
        return rc;
    }
    net->d_nan_spans = (ach_nan_span *)mem;
    net->d_nan_flag = (int32_t *)((char *)mem + tb);
    net->n_nan_spans = k;
    return ACH_OK;
}

int an_finalize(an_network *net)
{
    if (!net || net->finalized || net->n == 0) return ACH_EINVAL;
    an_layer *last = net->layers[net->n - 1];
    net->classes = last->outputs;
    /* the layers below the last layer with stopbackward = 1 run forward only
     * and are not updated (NetworkFactory.c:881-893, 981-991: only the value
     * 1 counts there, while the backward loop stops at any nonzero value,
     * NNetwork.c:648) */
    int last_stop = -1;
    for (int i = 0; i < net->n; ++i)
        if (net->layers[i]->stopbackward == 1) last_stop = i;
    for (int k = 0; k < last_stop; ++k) {
        net->layers[k]->onlyforward = 1;
        net->layers[k]->train = 0;
    }
    /* a layer the backward loop skips writes no input delta: the layer
     * below then reads the delta the forward zeroed (NNetwork.c:388-391),
     * so that delta joins the region zeroed every forward pass           */
    for (int i = last_stop + 1; i < net->n; ++i) {
        const an_layer *l = net->layers[i];
        if (!l->onlyforward || l->shares_prev || i == 0) continue;
        int j = i - 1;
        while (j > 0 && net->layers[j]->shares_prev) --j;
        net->layers[j]->zero_delta = 1;
    }
    net->layer_opts = 0;
    for (int i = 0; i < net->n; ++i) {
        const an_layer *l = net->layers[i];
        if (l->stopbackward || l->onlyforward || !l->train || l->learning_rate_scale != 1.f)
            net->layer_opts = 1;
    }
    /* deltas the next layer accumulates into (+=) must start at zero:
     * avgpool / softmax backward add into their input delta.  Max-pool
     * backward writes its input delta outright (accumulate = 0), which is
     * the same as adding to the zeroed buffer.                             */
    for (int i = 1; i < net->n; ++i) {
        an_layer *l = net->layers[i];
        if (l->type == AN_AVGPOOL || l->type == AN_SOFTMAX) {
            int j = i - 1;
            while (j > 0 && net->layers[j]->shares_prev) --j;
            net->layers[j]->zero_delta = 1;
        }
    }
    /* flat parameter buffers use 64-float aligned per-layer slots */
    bump dry = {NULL, 0, 1};
    layout(net, &dry);
    size_t nw = 0, nb = 0;
    for (int i = 0; i < net->n; ++i) {
        an_layer *l = net->layers[i];
        if (l->type != AN_CONVOLUTIONAL) continue;
        nw += (size_t)((l->nweights + 63) & ~63);
        nb += (size_t)((l->n + 63) & ~63) * (l->batch_normalize ? 2 : 1);
    }
    const size_t extra = al(sizeof(float) * nw) * 4 + al(sizeof(float) * nb) * 2;
    net->arena_bytes = dry.off + extra;
    AN_CHECK(ach_malloc(&net->arena, net->arena_bytes));
    AN_CHECK(ach_stream_create(&net->stream));
    AN_CHECK(ach_stream_create(&net->wstream));
    net->ev_ready = (void **)calloc((size_t)(net->n > 0 ? net->n : 1), sizeof(void *));
    net->ev_dgrad = (void **)calloc((size_t)(net->n > 0 ? net->n : 1), sizeof(void *));
    if (!net->ev_ready || !net->ev_dgrad) return ACH_EINVAL;
    for (int i = 0; i < net->n; ++i) {
        if (net->layers[i]->type != AN_CONVOLUTIONAL) continue;
        AN_CHECK(ach_event_create(&net->ev_ready[i]));
        AN_CHECK(ach_event_create(&net->ev_dgrad[i]));
    }
    AN_CHECK(ach_event_create(&net->ev_joined));
    bump real = {(char *)net->arena, 0, 0};
    layout(net, &real);
    /* flat parameter buffers at the arena tail */
    char *tail = (char *)net->arena + real.off;
    net->wflat = (float *)tail;
    tail += al(sizeof(float) * nw);
    net->vflat = (float *)tail;
    tail += al(sizeof(float) * nw);
    net->bflat = (float *)tail;
    tail += al(sizeof(float) * nb);
    net->bvflat = (float *)tail;
    tail += al(sizeof(float) * nb);
    net->wtflat = (float *)tail;
    tail += al(sizeof(float) * nw);
    net->wftflat = (float *)tail;
    net->nweights_total = nw;
    net->nbias_total = nb;
    size_t ow = 0, ob = 0;
    for (int i = 0; i < net->n; ++i) {
        an_layer *l = net->layers[i];
        if (l->type != AN_CONVOLUTIONAL) continue;
        l->weights = net->wflat + ow;
        l->weight_updates = net->vflat + ow;
        /* fully connected geometry: the forward GEMM reads W itself */
        const ach_conv_desc dl = conv_desc(l);
        l->weights_kmajor = ach_conv_is_fully_connected(&dl) ? l->weights : net->wtflat + ow;
        l->weights_flipped = net->wftflat + ow;
        ow += (size_t)((l->nweights + 63) & ~63);
        l->biases = net->bflat + ob;
        l->bias_updates = net->bvflat + ob;
        ob += (size_t)((l->n + 63) & ~63);
        if (l->batch_normalize) {
            l->scales = net->bflat + ob;
            l->scale_updates = net->bvflat + ob;
            ob += (size_t)((l->n + 63) & ~63);
        } else {
            l->scales = l->scale_updates = NULL;
        }
    }
    /* filter-layout jobs: the flipped copy only where an input gradient is
     * computed (not for the first layer, whose state.delta is NULL) */
    net->jobs = (ach_filter_job *)calloc((size_t)(net->n > 0 ? net->n : 1),
                                         sizeof(ach_filter_job));
    if (!net->jobs) return ACH_EINVAL;
    net->njobs = 0;
    for (int i = 0; i < net->n; ++i) {
        an_layer *l = net->layers[i];
        if (l->type != AN_CONVOLUTIONAL) continue;
        ach_filter_job *j = &net->jobs[net->njobs++];
        j->desc = conv_desc(l);
        j->w = l->weights;
        j->wt = l->weights_kmajor;
        j->wft = i > 0 ? l->weights_flipped : NULL;
    }
    AN_CHECK(setup_nan_scan(net));
    /* zero everything once (momentum buffers, biases, stats, deltas) */
    AN_CHECK(ach_fill((float *)net->arena, net->arena_bytes / sizeof(float), 0.f, net->stream));
    for (int i = 0; i < net->n; ++i) {
        an_layer *l = net->layers[i];
        if (l->type != AN_CONVOLUTIONAL) continue;
        AN_CHECK(ach_memcpy_h2d(l->weights, net->init_w[i], sizeof(float) * l->nweights,
                                net->stream));
        free(net->init_w[i]);
        net->init_w[i] = NULL;
        if (l->batch_normalize) /* ScaleData.init(1.0) */
            AN_CHECK(ach_fill(l->scales, (size_t)l->n, 1.f, net->stream));
    }
    AN_CHECK(ach_stream_sync(net->stream));
    net->finalized = 1;
    return ACH_OK;
}

void an_free(an_network *net)
{
    if (!net) return;
    for (int i = 0; i < net->n; ++i) {
        if (net->init_w) free(net->init_w[i]);
        free(net->layers[i]);
    }
    free(net->layers);
    free(net->init_w);
    free(net->jobs);
    if (net->wstream) ach_stream_sync(net->wstream);
    if (net->stream) ach_stream_sync(net->stream);
    free(net->steps);
    free(net->scales);
    if (net->ev_ready) {
        for (int i = 0; i < net->n; ++i)
            if (net->ev_ready[i]) ach_event_destroy(net->ev_ready[i]);
        free(net->ev_ready);
    }
    if (net->ev_dgrad) {
        for (int i = 0; i < net->n; ++i)
            if (net->ev_dgrad[i]) ach_event_destroy(net->ev_dgrad[i]);
        free(net->ev_dgrad);
    }
    if (net->ev_joined) ach_event_destroy(net->ev_joined);
    ach_free(net->d_nan_spans);
    ach_free(net->arena);
    if (net->wstream) ach_stream_destroy(net->wstream);
    ach_stream_destroy(net->stream);
    free(net);
}

/* ======================================================================== */
ach_stream_t an_stream(an_network *net) { return net->stream; }

int an_set_input(an_network *net, const float *host_input, const float *host_truth)
{
    if (!net || !net->finalized || !host_input) return ACH_EINVAL;
    AN_CHECK(ach_memcpy_h2d(net->input, host_input, sizeof(float) * net->batch * net->inputs,
                            net->stream));
    if (host_truth)
        AN_CHECK(ach_memcpy_h2d(net->truth, host_truth,
                                sizeof(float) * net->batch * net->classes, net->stream));
    return ACH_OK;
}

int an_set_input_device(an_network *net, const float *dev_input, const float *dev_truth)
{
    if (!net || !net->finalized || !dev_input) return ACH_EINVAL;
    AN_CHECK(ach_memcpy_d2d(net->input, dev_input, sizeof(float) * net->batch * net->inputs,
                            net->stream));
    if (dev_truth)
        AN_CHECK(ach_memcpy_d2d(net->truth, dev_truth,
                                sizeof(float) * net->batch * net->classes, net->stream));
    return ACH_OK;
}

static an_state base_state(an_network *net)
{
    an_state st;
    st.truth = net->truth;
    st.input = net->input;
    st.delta = NULL;
    st.workspace = net->workspace;
    st.workspace_bytes = net->workspace_bytes;
    st.train = 1;
    st.index = 0;
    return st;
}

/* NNetwork.forward (NNetwork.c:382-396): deltas start at zero, then every
 * layer runs with state.input = previous output.                           */
int an_forward(an_network *net, int train)
{
    if (!net || !net->finalized) return ACH_EINVAL;
    an_state st = base_state(net);
    st.train = train;
    if (!train) st.truth = NULL; /* NNetwork.predict: state.truth = 0 */
    /* the filter layouts the conv GEMMs read, from the current weights */
    AN_CHECK(ach_conv_prepare_filters(net->njobs, net->jobs, net->stream));
    if (train && net->zero_floats)
        AN_CHECK(ach_fill(net->zero_region, net->zero_floats, 0.f, net->stream));
    int rc = ACH_OK;
    for (int i = 0; i < net->n && rc == ACH_OK; ++i) {
        an_layer *l = net->layers[i];
        st.index = i;
        rc = l->forward(net, l, st);
        st.input = l->output;
    }
    return rc;
}

static an_state backward_state(an_network *net, int i)
{
    an_state st = base_state(net);
    st.index = i;
    if (i > 0) {
        st.input = net->layers[i - 1]->output;
        st.delta = net->layers[i - 1]->delta;
    }
    return st;
}

/* NNetwork.backward (NNetwork.c:627-654).                                 */
/* the main stream waits for every weight gradient enqueued so far */
static int join_wgrad(an_network *net)
{
    AN_CHECK(ach_event_record(net->ev_joined, net->wstream));
    return ach_stream_wait_event(net->stream, net->ev_joined);
}

int an_backward(an_network *net)
{
    if (!net || !net->finalized) return ACH_EINVAL;
    net->in_chain = 1;
    int rc = ACH_OK;
    for (int i = net->n - 1; i >= 0 && rc == ACH_OK; --i) {
        an_layer *l = net->layers[i];
        if (l->stopbackward) break; /* NNetwork.c:648-651 */
        if (l->onlyforward) continue;
        rc = l->backward(net, l, backward_state(net, i));
    }
    net->in_chain = 0;
    for (int i = 0; i < net->n; ++i) {
        net->layers[i]->grad_applied = 0;
        net->layers[i]->planes_ready = 0;
    }
    AN_CHECK(rc);
    return join_wgrad(net);
}

/* One layer of the loops above, with the same NetworkState: the
 * reference's per-layer NLayer.forward / backward entry points.           */
int an_layer_forward(an_network *net, int i, int train)
{
    an_layer *l = an_get_layer(net, i);
    if (!l || !net->finalized) return ACH_EINVAL;
    an_state st = base_state(net);
    st.train = train;
    st.index = i;
    if (i > 0) st.input = net->layers[i - 1]->output;
    if (l->type == AN_CONVOLUTIONAL)
        AN_CHECK(ach_conv_prepare_filters(net->njobs, net->jobs, net->stream));
    if (train && l->zero_delta && !l->shares_prev)
        AN_CHECK(ach_fill(l->delta, (size_t)l->batch * l->outputs, 0.f, net->stream));
    return l->forward(net, l, st);
}

int an_layer_backward(an_network *net, int i)
{
    an_layer *l = an_get_layer(net, i);
    if (!l || !net->finalized) return ACH_EINVAL;
    if (l->type == AN_CONVOLUTIONAL)
        AN_CHECK(ach_conv_prepare_filters(net->njobs, net->jobs, net->stream));
    AN_CHECK(l->backward(net, l, backward_state(net, i)));
    return join_wgrad(net);
}

/* NNetwork.updateCPU (NNetwork.c:667-680): every conv layer's update with
 * update batch = batch * subdivisions, as two launches over the flat
 * buffers.                                                                 */
static int update_at_rate(an_network *net, float rate)
{
    const int batch = net->batch * net->subdivisions;
    if (net->layer_opts) {
        /* layer by layer: frozen layers skip, the rest at rate * their scale
         * (updateCPU NNetwork.c:667-680; ConvolutionalLayer.c:959-960) */
        for (int i = 0; i < net->n; ++i) {
            an_layer *l = net->layers[i];
            if (l->type != AN_CONVOLUTIONAL || !l->train) continue;
            AN_CHECK(conv_update(net, l, batch, rate * l->learning_rate_scale, net->momentum,
                                 net->decay));
        }
        return ACH_OK;
    }
    const float a1 = -net->decay * batch;
    const float a2 = rate / batch;
    AN_CHECK(ach_sgd_update(net->nweights_total, net->wflat, net->vflat, a1, a2, net->momentum,
                            net->stream));
    return ach_sgd_update(net->nbias_total, net->bflat, net->bvflat, 0.f, a2, net->momentum,
                          net->stream);
}

float an_current_rate(an_network *net)
{
    return an_rate(net, net->seen / ((uint64_t)net->batch * (uint64_t)net->subdivisions));
}

int an_update(an_network *net)
{
    if (!net || !net->finalized) return ACH_EINVAL;
    return update_at_rate(net, an_current_rate(net));
}

/* NNetwork.predict (NNetwork.c:411-422): forward with train = 0 (BN on the
 * rolling statistics, dropout off, no truth) on a host batch; the output of
 * the last layer (NNetwork.getOutput, NNetwork.c:400-407; this build has no
 * cost layers), batch x outputs floats, is copied to host_output.          */
int an_predict(an_network *net, const float *host_input, float *host_output)
{
    if (!net || !net->finalized || !host_input || !host_output) return ACH_EINVAL;
    AN_CHECK(an_set_input(net, host_input, NULL));
    AN_CHECK(an_forward(net, 0));
    const an_layer *last = net->layers[net->n - 1];
    return ach_memcpy_d2h(host_output, last->output,
                          sizeof(float) * (size_t)last->batch * last->outputs, net->stream);
}

/* NNetwork.fuseConvBatchnorm (NNetwork.c:272-288), conv layers: each BN conv
 * layer's inference BN is folded into its filters and biases
 * (ach_conv_bn_fold, ConvolutionalLayer.c:983-1003) and the layer becomes a
 * plain conv layer with bias (batch_normalize = 0).  The reference calls it
 * after loading weights for validation (Classifier.c:369-373); a saved file
 * afterwards holds no BN arrays for these layers, as in the reference.      */
int an_fuse_conv_batchnorm(an_network *net)
{
    if (!net || !net->finalized) return ACH_EINVAL;
    for (int i = 0; i < net->n; ++i) {
        an_layer *l = net->layers[i];
        if (l->type != AN_CONVOLUTIONAL || !l->batch_normalize) continue;
        AN_CHECK(ach_conv_bn_fold(l->n, l->nweights / l->n, l->weights, l->biases, l->scales,
                                  l->rolling_mean, l->rolling_variance, net->stream));
        l->batch_normalize = 0;
    }
    return ach_stream_sync(net->stream);
}

/* DnnUtils.topK (DnnUtils.c:463-477): indices of the k largest of a[0..n),
 * largest first (insertion with strict '>', so equal values keep the order
 * in which the insertion left them, as in the reference).                  */
void an_top_k(const float *a, int n, int k, int *index)
{
    for (int j = 0; j < k; ++j) index[j] = -1;
    for (int i = 0; i < n; ++i) {
        int curr = i;
        for (int j = 0; j < k; ++j) {
            if (index[j] < 0 || a[curr] > a[index[j]]) {
                const int t = curr;
                curr = index[j];
                index[j] = t;
            }
        }
    }
}

/* the kernels of one training step: forward, both backward streams and
 * the update                                                               */
static int enqueue_step(an_network *net, int update, float rate)
{
    AN_CHECK(an_forward(net, 1));
    /* with an update, each layer's is enqueued by its backward (the join at
     * the end of an_backward waits for them); with layer options some
     * layers run no backward, so the updates follow the loop instead */
    net->early_update = update && !net->layer_opts;
    net->early_rate = rate;
    const int rc = an_backward(net);
    net->early_update = 0;
    AN_CHECK(rc);
    if (update && net->layer_opts) AN_CHECK(update_at_rate(net, rate));
    return ach_nan_scan(net->d_nan_spans, net->n_nan_spans, net->d_nan_flag, net->stream);
}

/* One minibatch of NNetwork.train(ImageData) (NNetwork.c:762-805, with
 * NNetwork.train(input, truth) at :740-758): seen += batch, forward,
 * backward; after every subdivisions-th minibatch cur_iteration += 1 and
 * the update at the policy's rate.                                        */
int an_train_step(an_network *net)
{
    if (!net || !net->finalized) return ACH_EINVAL;
    net->dropout_step = (uint32_t)(net->seen / (uint64_t)net->batch);
    net->seen += (uint64_t)net->batch;
    const int update = (net->seen / (uint64_t)net->batch) % (uint64_t)net->subdivisions == 0;
    const float rate = update ? an_current_rate(net) : 0.f;
    AN_CHECK(enqueue_step(net, update, rate));
    if (update) net->cur_iteration += 1;
    return ACH_OK;
}

int an_nan_status(an_network *net, int *layer, int *what)
{
    if (!net || !net->finalized) return ACH_EINVAL;
    int32_t f = INT32_MAX;
    if (net->d_nan_flag) AN_CHECK(ach_memcpy_d2h(&f, net->d_nan_flag, sizeof(f), net->stream));
    if (f == INT32_MAX) return 0;
    if (layer) *layer = f / 4;
    if (what) *what = f % 4;
    return 1;
}

int an_get_loss(an_network *net, float *loss)
{
    if (!net || !net->finalized || !loss) return ACH_EINVAL;
    int nl = -1, nw = 0;
    const int nan = an_nan_status(net, &nl, &nw);
    if (nan < 0) return nan;
    if (nan) {
        static const char *what[4] = {"mean", "variance", "scales", "scale updates"};
        fprintf(stderr, "an_get_loss: layer %d: NaN in its batch-norm %s (the reference's CPU "
                "path exits here, %s)\n", nl, what[nw],
                nw < 2 ? "NormData.c:273-276" : "ScaleData.c:51-54, 67-70");
        return ACH_ENAN;
    }
    float sum = 0;
    int count = 0;
    for (int i = 0; i < net->n; ++i) {
        an_layer *l = net->layers[i];
        if (l->type != AN_SOFTMAX) continue;
        float c = 0;
        AN_CHECK(ach_memcpy_d2h(&c, l->cost, sizeof(float), net->stream));
        sum += c;
        ++count;
    }
    /* getNetworkCost (NNetwork.c:611-624), then / (subdivisions*batch) */
    const float cost = count ? sum / count : 0.f;
    *loss = cost / net->batch;
    if (isnan(*loss)) return ACH_ENAN; /* the CPU path aborts on NaN */
    return ACH_OK;
}

int an_train(an_network *net, const float *host_input, const float *host_truth, float *loss)
{
    AN_CHECK(an_set_input(net, host_input, host_truth));
    AN_CHECK(an_train_step(net));
    return an_get_loss(net, loss);
}

/* ======================================================================== */
int an_n_layers(const an_network *net) { return net ? net->n : 0; }
an_layer *an_get_layer(an_network *net, int i)
{
    return (net && i >= 0 && i < net->n) ? net->layers[i] : NULL;
}
int an_layer_shape(const an_network *net, int i, int *out)
{
    if (!net || i < 0 || i >= net->n || !out) return ACH_EINVAL;
    const an_layer *l = net->layers[i];
    out[0] = (int)l->type;
    out[1] = l->out_c;
    out[2] = l->out_h;
    out[3] = l->out_w;
    out[4] = l->c;
    out[5] = l->h;
    out[6] = l->w;
    out[7] = l->batch;
    return ACH_OK;
}

int an_batch(const an_network *net) { return net->batch; }
float *an_input(an_network *net) { return net->input; }
float *an_truth(an_network *net) { return net->truth; }
int an_classes(const an_network *net) { return net->classes; }
uint64_t an_seen(const an_network *net) { return net->seen; }
int an_iteration(const an_network *net) { return net->cur_iteration; }

void *an_layer_buffer(an_network *net, int li, int which, size_t *count)
{
    *count = 0;
    an_layer *l = an_get_layer(net, li);
    if (!l) return NULL;
    const size_t bo = (size_t)l->batch * l->outputs;
    void *p = NULL;
    size_t n = 0;
    switch (which) {
    case 0: p = l->output; n = bo; break;
    case 1: p = l->delta; n = bo; break;
    case 2: p = l->weights; n = (size_t)l->nweights; break;
    case 3: p = l->weight_updates; n = (size_t)l->nweights; break;
    case 4: p = l->biases; n = (size_t)l->n; break;
    case 5: p = l->bias_updates; n = (size_t)l->n; break;
    case 6: p = l->scales; n = (size_t)l->n; break;
    case 7: p = l->scale_updates; n = (size_t)l->n; break;
    case 8: p = l->rolling_mean; n = (size_t)l->n; break;
    case 9: p = l->rolling_variance; n = (size_t)l->n; break;
    case 10: p = l->mean; n = (size_t)l->n; break;
    case 11: p = l->variance; n = (size_t)l->n; break;
    case 12: p = l->x; n = bo; break;
    case 14: p = l->indexes; n = bo; break;
    case 15: p = l->loss; n = bo; break;
    default: break;
    }
    if (p) *count = n;
    return p;
}

double an_step_conv_gflop(const an_network *net)
{
    double tot = 0;
    for (int i = 0; i < net->n; ++i) {
        const an_layer *l = net->layers[i];
        if (l->type != AN_CONVOLUTIONAL) continue;
        const double f = 2.0 * l->batch * l->n * l->out_h * l->out_w * (double)l->c * l->size *
                         l->size;
        tot += f * (i == 0 ? 2 : 3); /* layer 0 has no input gradient */
    }
    return tot / 1e9;
}

/* ======================================================================== */
/* Darknet .weights files (NNetwork.loadWeights / saveWeightsUpto,
 * NNetwork.c:64-151; per layer ConvolutionalLayer.saveWeights / loadWeights,
 * ConvolutionalLayer.c:422-486).  Little-endian:
 *   int32 major = 0, minor = 2, revision = 5; uint64 seen;
 *   for each convolutional layer in order:
 *     biases[n], (batch_normalize: scales[n], rolling_mean[n],
 *     rolling_variance[n]), weights[nweights]  (float32 each)
 * Save writes seen = cur_iteration * batch * subdivisions and, as the
 * reference does (NNetwork.c:125), makes that the network's seen; load
 * sets cur_iteration = seen / (batch * subdivisions) (NNetwork.c:88).     */

/* one conv layer's parameter arrays in file order */
static int conv_param_arrays(an_layer *l, float **ptr, size_t *cnt)
{
    int k = 0;
    if (l->connected) {
        /* darknet's connected-layer order: biases, weights, then BN arrays */
        ptr[k] = l->biases; cnt[k++] = (size_t)l->n;
        ptr[k] = l->weights; cnt[k++] = (size_t)l->nweights;
        if (l->batch_normalize) {
            ptr[k] = l->scales; cnt[k++] = (size_t)l->n;
            ptr[k] = l->rolling_mean; cnt[k++] = (size_t)l->n;
            ptr[k] = l->rolling_variance; cnt[k++] = (size_t)l->n;
        }
        return k;
    }
    ptr[k] = l->biases; cnt[k++] = (size_t)l->n;
    if (l->batch_normalize) {
        ptr[k] = l->scales; cnt[k++] = (size_t)l->n;
        ptr[k] = l->rolling_mean; cnt[k++] = (size_t)l->n;
        ptr[k] = l->rolling_variance; cnt[k++] = (size_t)l->n;
    }
    ptr[k] = l->weights; cnt[k++] = (size_t)l->nweights;
    return k;
}

int an_save_weights(an_network *net, const char *path)
{
    if (!net || !net->finalized || !path) return ACH_EINVAL;
    FILE *fp = fopen(path, "wb");
    if (!fp) {
        fprintf(stderr, "an_save_weights: cannot open %s\n", path);
        return ACH_EINVAL;
    }
    const int32_t hdr[3] = {0, 2, 5};
    const uint64_t seen =
        (uint64_t)net->cur_iteration * (uint64_t)net->batch * (uint64_t)net->subdivisions;
    net->seen = seen;
    int rc = ACH_OK;
    if (fwrite(hdr, sizeof(int32_t), 3, fp) != 3 || fwrite(&seen, sizeof(seen), 1, fp) != 1)
        rc = ACH_EINVAL;
    float *host = NULL;
    size_t host_cap = 0;
    for (int i = 0; i < net->n && rc == ACH_OK; ++i) {
        an_layer *l = net->layers[i];
        if (l->type != AN_CONVOLUTIONAL) continue;
        float *ptr[5];
        size_t cnt[5];
        const int na = conv_param_arrays(l, ptr, cnt);
        for (int a = 0; a < na && rc == ACH_OK; ++a) {
            if (cnt[a] > host_cap) {
                float *nh = (float *)realloc(host, cnt[a] * sizeof(float));
                if (!nh) { rc = ACH_EINVAL; break; }
                host = nh;
                host_cap = cnt[a];
            }
            rc = ach_memcpy_d2h(host, ptr[a], cnt[a] * sizeof(float), net->stream);
            if (rc == ACH_OK && fwrite(host, sizeof(float), cnt[a], fp) != cnt[a])
                rc = ACH_EINVAL;
        }
    }
    free(host);
    if (fclose(fp) != 0 && rc == ACH_OK) rc = ACH_EINVAL;
    return rc;
}

/* ConvolutionalLayer.transposeMatrix (ConvolutionalLayer.c:443-453): a is
 * rows x cols row-major on entry, cols x rows on return.                  */
static int transpose_host(float *a, int rows, int cols)
{
    float *t = (float *)malloc(sizeof(float) * (size_t)rows * cols);
    if (!t) return ACH_EINVAL;
    for (int x = 0; x < rows; ++x)
        for (int y = 0; y < cols; ++y) t[(size_t)y * rows + x] = a[(size_t)x * cols + y];
    memcpy(a, t, sizeof(float) * (size_t)rows * cols);
    free(t);
    return ACH_OK;
}

/* Reads as the reference does: a version >= 0.2 header carries a 64-bit
 * seen (older files none); layers are filled in order until the file ends,
 * a short array keeps the values it read (the rest unchanged) with a
 * warning.  Sets seen and the iteration (seen / batch).  A dontload layer
 * is skipped without reading (NNetwork.c:93-94), a dontloadscales layer
 * reads no BN arrays (ConvolutionalLayer.c:467), a flipped layer's weights
 * are transposed from [C*k*k][n] after the read (ConvolutionalLayer.c:
 * 483-485), and a header with major or minor above 1000 transposes the
 * weights of connected layers from [inputs][outputs] (darknet's
 * load_connected_weights; NNetwork.c:90 computes the flag).               */
int an_load_weights(an_network *net, const char *path)
{
    if (!net || !net->finalized || !path) return ACH_EINVAL;
    FILE *fp = fopen(path, "rb");
    if (!fp) {
        fprintf(stderr, "an_load_weights: cannot open %s\n", path);
        return ACH_EINVAL;
    }
    int32_t hdr[3];
    if (fread(hdr, sizeof(int32_t), 3, fp) != 3) {
        fclose(fp);
        return ACH_EINVAL;
    }
    if (hdr[0] * 10 + hdr[1] >= 2) {
        uint64_t seen = 0;
        if (fread(&seen, sizeof(seen), 1, fp) != 1) {
            fclose(fp);
            return ACH_EINVAL;
        }
        net->seen = seen;
    }
    const int transpose = hdr[0] > 1000 || hdr[1] > 1000;
    net->cur_iteration = (int)(net->seen / ((uint64_t)net->batch * net->subdivisions));
    int rc = ACH_OK;
    float *host = NULL;
    size_t host_cap = 0;
    for (int i = 0; i < net->n && rc == ACH_OK && !feof(fp); ++i) {
        an_layer *l = net->layers[i];
        if (l->type != AN_CONVOLUTIONAL || l->dontload) continue;
        float *ptr[5];
        size_t cnt[5];
        const int na = conv_param_arrays(l, ptr, cnt);
        for (int a = 0; a < na && rc == ACH_OK; ++a) {
            const int is_w = ptr[a] == l->weights;
            const int is_bn = ptr[a] == l->scales || ptr[a] == l->rolling_mean ||
                              ptr[a] == l->rolling_variance;
            if (is_bn && l->dontloadscales) continue;
            if (cnt[a] > host_cap) {
                float *nh = (float *)realloc(host, cnt[a] * sizeof(float));
                if (!nh) { rc = ACH_EINVAL; break; }
                host = nh;
                host_cap = cnt[a];
            }
            const size_t got = fread(host, sizeof(float), cnt[a], fp);
            if (got > 0 && got < cnt[a])
                fprintf(stderr, "an_load_weights: unexpected end of weights file at layer %d\n",
                        i);
            /* the flipped / transposed weights: whole-array transposes over
             * what was read and, past a short read, the values kept */
            const int fl = is_w && (l->connected ? transpose : l->flipped);
            if (fl) {
                if (got < cnt[a]) {
                    float *keep = (float *)malloc(sizeof(float) * cnt[a]);
                    if (!keep) { rc = ACH_EINVAL; break; }
                    rc = ach_memcpy_d2h(keep, ptr[a], cnt[a] * sizeof(float), net->stream);
                    if (rc == ACH_OK)
                        memcpy(host + got, keep + got, (cnt[a] - got) * sizeof(float));
                    free(keep);
                    if (rc != ACH_OK) break;
                }
                /* conv: [C*k*k][n] -> [n][C*k*k]; connected: [inputs][outputs] */
                rc = transpose_host(host, l->nweights / l->n, l->n);
                if (rc == ACH_OK)
                    rc = ach_memcpy_h2d(ptr[a], host, cnt[a] * sizeof(float), net->stream);
                continue;
            }
            if (got > 0) rc = ach_memcpy_h2d(ptr[a], host, got * sizeof(float), net->stream);
        }
    }
    free(host);
    fclose(fp);
    return rc;
}
