/*
 * oracle.c -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.
 *
 * Plain-C restatement of the reference CPU path (onlineaet/aet-cnn, AET-C).
 * The reference cannot be compiled here (it needs the AET compiler and its
 * runtime libraries), so each routine below restates the cited reference
 * lines in C.  Paths are relative to /root/reference/src/com/ai/dnn/.
 * Built with the reference's flags (-O3 -ffast-math -fopenmp, src/makefile:50)
 * except that -march is pinned to x86-64-v3 so the library runs on any AVX2
 * host.  Used only by tests/, __graft_entry__.smoke() and bench.py's CPU
 * baseline.
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int g_gemm_parallel = 0;
void or_set_gemm_parallel(int on) { g_gemm_parallel = on ? 1 : 0; }
int or_get_gemm_parallel(void) { return g_gemm_parallel; }
int or_max_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------------ */
/* GEMM: Gemm.c:53-66 (NN), :68-82 (NT), :84-97 (TN), :99-113 (TT),
 * driver Gemm.c:116-144 (BETA pre-scale then one call per row t).          */
static void gemm_nn(int M, int N, int K, float ALPHA, const float *A, int lda,
                    const float *B, int ldb, float *C, int ldc)
{
    for (int i = 0; i < M; ++i)
        for (int k = 0; k < K; ++k) {
            register float A_PART = ALPHA * A[i * lda + k];
            for (int j = 0; j < N; ++j)
                C[i * ldc + j] += A_PART * B[k * ldb + j];
        }
}

static void gemm_nt(int M, int N, int K, float ALPHA, const float *A, int lda,
                    const float *B, int ldb, float *C, int ldc)
{
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < N; ++j) {
            register float sum = 0;
            for (int k = 0; k < K; ++k)
                sum += ALPHA * A[i * lda + k] * B[j * ldb + k];
            C[i * ldc + j] += sum;
        }
}

static void gemm_tn(int M, int N, int K, float ALPHA, const float *A, int lda,
                    const float *B, int ldb, float *C, int ldc)
{
    for (int i = 0; i < M; ++i)
        for (int k = 0; k < K; ++k) {
            register float A_PART = ALPHA * A[k * lda + i];
            for (int j = 0; j < N; ++j)
                C[i * ldc + j] += A_PART * B[k * ldb + j];
        }
}

static void gemm_tt(int M, int N, int K, float ALPHA, const float *A, int lda,
                    const float *B, int ldb, float *C, int ldc)
{
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < N; ++j) {
            register float sum = 0;
            for (int k = 0; k < K; ++k)
                sum += ALPHA * A[i + k * lda] * B[k + j * ldb];
            C[i * ldc + j] += sum;
        }
}

void or_gemm(int TA, int TB, int M, int N, int K, float ALPHA,
             const float *A, int lda, const float *B, int ldb,
             float BETA, float *C, int ldc)
{
    if (BETA != 1) {
        for (int i = 0; i < M; ++i)
            for (int j = 0; j < N; ++j)
                C[i * ldc + j] *= BETA;
    }
    int t;
#pragma omp parallel for if (g_gemm_parallel) schedule(static)
    for (t = 0; t < M; ++t) {
        if (!TA && !TB)
            gemm_nn(1, N, K, ALPHA, A + t * lda, lda, B, ldb, C + t * ldc, ldc);
        else if (TA && !TB)
            gemm_tn(1, N, K, ALPHA, A + t, lda, B, ldb, C + t * ldc, ldc);
        else if (!TA && TB)
            gemm_nt(1, N, K, ALPHA, A + t * lda, lda, B, ldb, C + t * ldc, ldc);
        else
            gemm_tt(1, N, K, ALPHA, A + t, lda, B, ldb, C + t * ldc, ldc);
    }
}

/* ------------------------------------------------------------------------ */
/* im2col / col2im: Im2Col.c:65-103 and :155-192 (Caffe ext variants).
 * col2im zeroes the destination first (Im2Col.c:162).                      */
static inline int in_range(int a, int b) { return (unsigned)a < (unsigned)b; }

void or_im2col(const float *data_im, int channels, int height, int width,
               int kernel_h, int kernel_w, int pad_h, int pad_w,
               int stride_h, int stride_w, int dilation_h, int dilation_w,
               float *data_col)
{
    const int output_h = (height + 2 * pad_h - (dilation_h * (kernel_h - 1) + 1)) / stride_h + 1;
    const int output_w = (width + 2 * pad_w - (dilation_w * (kernel_w - 1) + 1)) / stride_w + 1;
    const int channel_size = height * width;
    for (int channel = channels; channel--; data_im += channel_size) {
        for (int kr = 0; kr < kernel_h; kr++) {
            for (int kc = 0; kc < kernel_w; kc++) {
                int input_row = -pad_h + kr * dilation_h;
                for (int orow = output_h; orow; orow--) {
                    if (!in_range(input_row, height)) {
                        for (int ocol = output_w; ocol; ocol--)
                            *(data_col++) = 0;
                    } else {
                        int input_col = -pad_w + kc * dilation_w;
                        for (int ocol = output_w; ocol; ocol--) {
                            *(data_col++) = in_range(input_col, width)
                                                ? data_im[input_row * width + input_col]
                                                : 0;
                            input_col += stride_w;
                        }
                    }
                    input_row += stride_h;
                }
            }
        }
    }
}

void or_col2im(const float *data_col, int channels, int height, int width,
               int kernel_h, int kernel_w, int pad_h, int pad_w,
               int stride_h, int stride_w, int dilation_h, int dilation_w,
               float *data_im)
{
    memset(data_im, 0, sizeof(float) * (size_t)height * width * channels);
    const int output_h = (height + 2 * pad_h - (dilation_h * (kernel_h - 1) + 1)) / stride_h + 1;
    const int output_w = (width + 2 * pad_w - (dilation_w * (kernel_w - 1) + 1)) / stride_w + 1;
    const int channel_size = height * width;
    for (int channel = channels; channel--; data_im += channel_size) {
        for (int kr = 0; kr < kernel_h; kr++) {
            for (int kc = 0; kc < kernel_w; kc++) {
                int input_row = -pad_h + kr * dilation_h;
                for (int orow = output_h; orow; orow--) {
                    if (!in_range(input_row, height)) {
                        data_col += output_w;
                    } else {
                        int input_col = -pad_w + kc * dilation_w;
                        for (int ocol = output_w; ocol; ocol--) {
                            if (in_range(input_col, width))
                                data_im[input_row * width + input_col] += *data_col;
                            data_col++;
                            input_col += stride_w;
                        }
                    }
                    input_row += stride_h;
                }
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Convolution GEMM parts: ConvolutionalLayer.c:337-344 (out size),
 * :684-803 (forward, fp32 branch), :906-947 (backward loop).               */
static int stride_h(const or_conv_shape *s) { return s->stride_y > 0 ? s->stride_y : s->stride; }
int or_conv_out_h(const or_conv_shape *s) { return (s->h + 2 * s->pad - s->size) / stride_h(s) + 1; }
int or_conv_out_w(const or_conv_shape *s) { return (s->w + 2 * s->pad - s->size) / s->stride + 1; }

size_t or_conv_workspace_floats(const or_conv_shape *s)
{
    return (size_t)or_conv_out_h(s) * or_conv_out_w(s) * s->size * s->size * s->c;
}

void or_conv_forward(const or_conv_shape *s, const float *input, const float *weights,
                     float *output, float *workspace)
{
    const int out_h = or_conv_out_h(s), out_w = or_conv_out_w(s);
    const int m = s->n, k = s->size * s->size * s->c, n = out_h * out_w;
    memset(output, 0, sizeof(float) * (size_t)s->batch * m * n);
    for (int i = 0; i < s->batch; ++i) {
        const float *im = input + (size_t)i * s->c * s->h * s->w;
        const float *b = workspace;
        float *c = output + (size_t)i * n * m;
        /* (the reference tests stride_x alone here, ConvolutionalLayer.c:788,
         * and would read a 1x1 layer with stride_x 1 and stride_y > 1 as if
         * unstrided: that case takes im2col) */
        if (s->size == 1 && s->stride == 1 && stride_h(s) == 1) {
            b = im;
        } else {
            or_im2col(im, s->c, s->h, s->w, s->size, s->size, s->pad, s->pad,
                      stride_h(s), s->stride, 1, 1, workspace);
        }
        or_gemm(0, 0, m, n, k, 1, weights, k, b, n, 1, c, n);
    }
}

void or_conv_backward(const or_conv_shape *s, const float *input, const float *my_delta,
                      const float *weights, float *weight_updates, float *delta,
                      float *workspace)
{
    const int out_h = or_conv_out_h(s), out_w = or_conv_out_w(s);
    const int m = s->n, n = s->size * s->size * s->c, k = out_h * out_w;
    for (int i = 0; i < s->batch; ++i) {
        const float *a = my_delta + (size_t)i * m * k;
        float *b = workspace;
        const float *im = input + (size_t)i * s->c * s->h * s->w;
        or_im2col(im, s->c, s->h, s->w, s->size, s->size, s->pad, s->pad,
                  stride_h(s), s->stride, 1, 1, b);
        or_gemm(0, 1, m, n, k, 1, a, k, b, k, 1, weight_updates, n);
        if (delta) {
            or_gemm(1, 0, n, k, m, 1, weights, n, a, k, 0, workspace, k);
            or_col2im(workspace, s->c, s->h, s->w, s->size, s->size, s->pad, s->pad,
                      stride_h(s), s->stride, 1, 1, delta + (size_t)i * s->c * s->h * s->w);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* IOData.addBias (IOData.c:43-55), BiasData.calcGrad (BiasData.c:40-57)
 * with DnnUtils.sum (DnnUtils.c:113-119).                                  */
void or_add_bias(float *output, const float *biases, int batch, int n, int spatial)
{
    for (int b = 0; b < batch; ++b)
        for (int i = 0; i < n; ++i)
            for (int j = 0; j < spatial; ++j)
                output[((size_t)b * n + i) * spatial + j] += biases[i];
}

static float dnn_sum(const float *a, int n)
{
    float sum = 0;
    for (int i = 0; i < n; ++i)
        sum += a[i];
    return sum;
}

void or_bias_grad(float *updates, const float *delta, int batch, int n, int spatial)
{
    for (int b = 0; b < batch; ++b)
        for (int i = 0; i < n; ++i)
            updates[i] += dnn_sum(delta + (size_t)spatial * (i + b * n), spatial);
}

/* ------------------------------------------------------------------------ */
/* Batch-norm forward, training: NormData.calcVarianceAndMean
 * (NormData.c:141-186), scalAxpyRollMeanAndRollVariance (:224-229),
 * normalize (:244-282).                                                    */
void or_bn_mean_var(const float *out, int batch, int channels, int spatial,
                    float *mean, float *variance)
{
    float *temp = (float *)calloc((size_t)batch * channels, sizeof(float));
    float *temp1 = (float *)calloc((size_t)batch * channels, sizeof(float));
    float *temp2 = (float *)calloc((size_t)batch * channels, sizeof(float));
    for (int i = 0; i < batch; ++i) {
        const float *item = out + (size_t)i * spatial * channels;
        for (int j = 0; j < channels; ++j)
            for (int k = 0; k < spatial; k++) {
                float value = item[(size_t)j * spatial + k];
                temp[i * channels + j] += value;
                temp1[i * channels + j] += (value * value);
                temp2[i * channels + j] += (-2 * value);
            }
    }
    float scale = 1. / (batch * spatial);
    for (int i = 0; i < channels; ++i) {
        mean[i] = 0;
        for (int j = 0; j < batch; ++j)
            mean[i] += temp[j * channels + i];
        mean[i] *= scale;
    }
    scale = 1. / (batch * spatial - 1);
    for (int i = 0; i < channels; ++i) {
        float t1 = 0, t2 = 0;
        for (int j = 0; j < batch; ++j) {
            t1 += temp1[j * channels + i];
            t2 += temp2[j * channels + i];
        }
        variance[i] = t1 + t2 * mean[i] + mean[i] * mean[i] * batch * spatial;
        variance[i] *= scale;
    }
    free(temp);
    free(temp1);
    free(temp2);
}

void or_bn_roll(int channels, const float *mean, const float *variance,
                float *rolling_mean, float *rolling_variance)
{
    /* scal_cpus / axpy_cpus take a float ALPHA (NormData.c:189-199) */
    const float keep = .9, take = .1;
    for (int i = 0; i < channels; ++i) rolling_mean[i] *= keep;
    for (int i = 0; i < channels; ++i) rolling_mean[i] += take * mean[i];
    for (int i = 0; i < channels; ++i) rolling_variance[i] *= keep;
    for (int i = 0; i < channels; ++i) rolling_variance[i] += take * variance[i];
}

static int f32_is_nan(float v)
{
    uint32_t u;
    memcpy(&u, &v, 4);
    return (u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu) != 0;
}

int or_bn_normalize(float *out, int batch, int channels, int spatial,
                    const float *mean, const float *variance,
                    const float *scales, const float *biases,
                    float *x, float *x_norm)
{
    int bad = 0;
    size_t size = (size_t)channels * spatial;
    float *inv = (float *)malloc(sizeof(float) * channels);
    for (int i = 0; i < channels; i++)
        inv[i] = 1.0 / (sqrt(variance[i]) + .000001f);
    for (int b = 0; b < batch; ++b) {
        float *o = out + b * size, *xn = x_norm + b * size, *xc = x + b * size;
        for (int f = 0; f < channels; ++f)
            for (int i = 0; i < spatial; i++) {
                size_t idx = (size_t)f * spatial + i;
                float value = o[idx];
                xc[idx] = value;
                value = (value - mean[f]) * inv[f];
                if (f32_is_nan(value)) bad = 1;
                xn[idx] = value;
                o[idx] = value * scales[f] + biases[f];
            }
    }
    free(inv);
    return bad;
}

void or_bn_normalize_roll(float *out, int batch, int channels, int spatial,
                          const float *rolling_mean, const float *rolling_variance,
                          const float *scales, const float *biases)
{
    size_t size = (size_t)channels * spatial;
    for (int f = 0; f < channels; ++f) {
        float inv = 1.0 / (sqrt(rolling_variance[f]) + .000001f);
        for (int b = 0; b < batch; ++b)
            for (int i = 0; i < spatial; i++) {
                float *o = out + b * size + (size_t)f * spatial + i;
                float v = (*o - rolling_mean[f]) * inv;
                *o = v * scales[f] + biases[f];
            }
    }
}

/* ConvolutionalLayer.fuseConvBatchnorm (ConvolutionalLayer.c:983-1003): fold
 * the inference BN of one conv layer into its filters and biases.  Per filter
 * f, with r = sqrt((double)rolling_variance[f] + 1e-5):
 *   biases[f]  <- biases[f] - scales[f] * rolling_mean[f] / r    (double)
 *   weights[f] <- weights[f] * (scales[f] / r)                   (double)
 * each rounded once to float.  Note the eps differs from normalizeByRoll's
 * 1/(sqrt(var) + 1e-6), as in the reference.                               */
void or_conv_bn_fold(int filters, int fsize, float *weights, float *biases,
                     const float *scales, const float *rolling_mean,
                     const float *rolling_variance)
{
    for (int f = 0; f < filters; ++f) {
        double r = sqrt((double)rolling_variance[f] + .00001);
        biases[f] = biases[f] - (double)scales[f] * rolling_mean[f] / r;
        double pre = scales[f] / r;
        for (int i = 0; i < fsize; ++i) weights[(size_t)f * fsize + i] *= pre;
    }
}

/* Batch-norm backward: backwardNormCPU (NLayer.c:246-278) =
 *   ScaleData.backwardScale (ScaleData.c:76-107), NData.scale (NData.c:238-248),
 *   DeltaData.calcMean (DeltaData.c:23-38), calcVariance (:41-58),
 *   normalize (:64-80).                                                    */
void or_bn_backward(float *delta, int batch, int filters, int spatial,
                    const float *x, const float *x_norm,
                    const float *mean, const float *variance,
                    const float *scales, float *scale_updates,
                    float *mean_delta, float *variance_delta)
{
    for (int f = 0; f < filters; ++f) {
        float sum = 0;
        for (int b = 0; b < batch; ++b)
            for (int i = 0; i < spatial; ++i) {
                size_t index = i + (size_t)spatial * (f + (size_t)filters * b);
                sum += delta[index] * x_norm[index];
            }
        scale_updates[f] += sum;
    }
    for (int b = 0; b < batch; ++b)
        for (int i = 0; i < filters; ++i)
            for (int j = 0; j < spatial; ++j)
                delta[((size_t)b * filters + i) * spatial + j] *= scales[i];
    for (int i = 0; i < filters; ++i) {
        mean_delta[i] = 0;
        for (int j = 0; j < batch; ++j)
            for (int k = 0; k < spatial; ++k)
                mean_delta[i] += delta[(size_t)j * filters * spatial + (size_t)i * spatial + k];
        mean_delta[i] *= (-1. / sqrt(variance[i] + .00001f));
    }
    for (int i = 0; i < filters; ++i) {
        variance_delta[i] = 0;
        for (int j = 0; j < batch; ++j)
            for (int k = 0; k < spatial; ++k) {
                size_t index = (size_t)j * filters * spatial + (size_t)i * spatial + k;
                variance_delta[i] += delta[index] * (x[index] - mean[i]);
            }
        variance_delta[i] *= -.5 * pow(variance[i] + .00001f, (float)(-3. / 2.));
    }
    for (int j = 0; j < batch; ++j)
        for (int f = 0; f < filters; ++f)
            for (int k = 0; k < spatial; ++k) {
                size_t index = (size_t)j * filters * spatial + (size_t)f * spatial + k;
                delta[index] = delta[index] * 1. / (sqrt(variance[f] + .00001f))
                             + variance_delta[f] * 2. * (x[index] - mean[f]) / (spatial * batch)
                             + mean_delta[f] / (spatial * batch);
            }
}

/* ------------------------------------------------------------------------ */
/* Activations: Activation.h:53 (linear), :56 (relu), :61 (leaky: .1*x in
 * double), :87/:99/:104 (gradients); Activation.c:160-179, :233-239.       */
static inline float leaky_activate(float x) { return (x > 0) ? x : .1 * x; }
static inline float relu_activate(float x) { return x * (x > 0); }
static inline float logistic_activate(float x) { return 1. / (1. + exp(-x)); }
static inline float leaky_gradient(float x) { return (x > 0) ? 1 : .1; }
static inline float relu_gradient(float x) { return (x > 0); }
static inline float logistic_gradient(float x) { return (1 - x) * x; }

void or_activate(float *x, int n, int act)
{
    int i;
    if (act == OR_LINEAR) return;
    if (act == OR_LEAKY) {
#pragma omp parallel for
        for (i = 0; i < n; ++i) x[i] = leaky_activate(x[i]);
    } else if (act == OR_RELU) {
        for (i = 0; i < n; ++i) x[i] = relu_activate(x[i]);
    } else if (act == OR_LOGISTIC) {
#pragma omp parallel for
        for (i = 0; i < n; ++i) x[i] = logistic_activate(x[i]);
    }
}

void or_gradient(const float *y, int n, int act, float *delta)
{
    int i;
#pragma omp parallel for
    for (i = 0; i < n; ++i) {
        float g = 1;
        if (act == OR_LEAKY) g = leaky_gradient(y[i]);
        else if (act == OR_RELU) g = relu_gradient(y[i]);
        else if (act == OR_LOGISTIC) g = logistic_gradient(y[i]);
        delta[i] *= g;
    }
}

/* ------------------------------------------------------------------------ */
/* Max-pool: MaxPoolLayer.c:40-41 (out size), :237-272 (forward, -FLT_MAX
 * init, strict >, global flat argmax), :318-331 (backward scatter-add).     */
int or_maxpool_out(int in, int size, int stride, int padding)
{
    return (in + padding - size) / stride + 1;
}

void or_maxpool_forward(const float *input, int batch, int c, int lh, int lw,
                        int size, int stride, int pad, float *output, int *indexes)
{
    or_maxpool_forward_xy(input, batch, c, lh, lw, size, stride, stride, pad, output, indexes);
}

void or_maxpool_forward_xy(const float *input, int batch, int c, int lh, int lw, int size,
                           int stride_x, int stride_y, int pad, float *output, int *indexes)
{
    const int w_offset = -pad / 2, h_offset = -pad / 2;
    const int h = or_maxpool_out(lh, size, stride_y, pad);
    const int w = or_maxpool_out(lw, size, stride_x, pad);
    for (int b = 0; b < batch; ++b)
        for (int k = 0; k < c; ++k)
            for (int i = 0; i < h; ++i)
                for (int j = 0; j < w; ++j) {
                    int out_index = j + w * (i + h * (k + c * b));
                    float max = -FLT_MAX;
                    int max_i = -1;
                    for (int n = 0; n < size; ++n)
                        for (int m = 0; m < size; ++m) {
                            int cur_h = h_offset + i * stride_y + n;
                            int cur_w = w_offset + j * stride_x + m;
                            int index = cur_w + lw * (cur_h + lh * (k + b * c));
                            int valid = (cur_h >= 0 && cur_h < lh && cur_w >= 0 && cur_w < lw);
                            float val = valid ? input[index] : -FLT_MAX;
                            max_i = (val > max) ? index : max_i;
                            max = (val > max) ? val : max;
                        }
                    output[out_index] = max;
                    if (indexes) indexes[out_index] = max_i;
                }
}

void or_maxpool_backward(const float *my_delta, const int *indexes, int total,
                         float *delta)
{
    for (int i = 0; i < total; ++i)
        delta[indexes[i]] += my_delta[i];
}

/* ------------------------------------------------------------------------ */
/* Global average pool: AvgPoolLayer.c:29-46 (forward), :73-88 (backward).   */
void or_avgpool_forward(const float *input, int batch, int c, int wh, float *output)
{
    for (int b = 0; b < batch; ++b)
        for (int k = 0; k < c; ++k) {
            int out_index = k + b * c;
            output[out_index] = 0;
            for (int i = 0; i < wh; ++i)
                output[out_index] += input[i + wh * (k + b * c)];
            output[out_index] /= wh;
        }
}

void or_avgpool_backward(const float *layer_delta, int batch, int c, int wh, float *delta)
{
    for (int b = 0; b < batch; ++b)
        for (int k = 0; k < c; ++k) {
            int out_index = k + b * c;
            for (int i = 0; i < wh; ++i)
                delta[i + wh * (k + b * c)] += layer_delta[out_index] / (wh);
        }
}

/* ------------------------------------------------------------------------ */
/* Softmax + cross-entropy: SoftMaxLayer.c:67-83 (softmax: float max, double
 * exp), :86-94 (softmax_cpu), :47-55 (xent), :99-119 (forwardCPU),
 * :291-316 (backward: axpy 1.0), NData.sum (NData.c:321-328).               */
static void softmax_1(const float *input, int n, float temp, float *output, int stride)
{
    float sum = 0;
    float largest = -FLT_MAX;
    for (int i = 0; i < n; ++i)
        if (input[i * stride] > largest) largest = input[i * stride];
    for (int i = 0; i < n; ++i) {
        float e = exp(input[i * stride] / temp - largest / temp);
        sum += e;
        output[i * stride] = e;
    }
    for (int i = 0; i < n; ++i) output[i * stride] /= sum;
}

float or_softmax_xent_forward(const float *input, int batch, int inputs, int groups,
                              float temperature, const float *truth,
                              float *output, float *delta, float *error)
{
    const int n = inputs / groups;
    for (int b = 0; b < batch; ++b)
        for (int g = 0; g < groups; ++g)
            softmax_1(input + (size_t)b * inputs + g * n, n, temperature,
                      output + (size_t)b * inputs + g * n, 1);
    if (!truth) return 0;
    const int total = batch * inputs;
    for (int i = 0; i < total; ++i) {
        float t = truth[i], p = output[i];
        error[i] = t ? -logf(p) : 0;
        delta[i] = t - p;
    }
    float sums = 0;
    for (int i = 0; i < total; ++i) sums += error[i];
    return sums;
}

void or_softmax_backward(const float *delta, int n, float *delta_prev)
{
    for (int i = 0; i < n; i++) delta_prev[i] += 1.0 * delta[i];
}

/* ------------------------------------------------------------------------ */
/* Dropout: DropoutLayer.c:55-86 (r < p -> 0, else x * 1/(1-p)).  The
 * reference draws r from the global rand() stream; a GPU cannot reproduce
 * that sequence, so r comes from a counter-based generator: the SplitMix64
 * finaliser (Steele, Lea, Flood 2014) over (seed, iteration, layer, index),
 * top 24 bits scaled to [0,1).                                             */
float or_dropout_uniform(uint64_t seed, uint32_t iter, uint32_t layer, uint32_t i)
{
    uint64_t z = seed + 0x9E3779B97F4A7C15ull * (((uint64_t)layer << 32) | iter);
    z ^= (uint64_t)i * 0xD1B54A32D192ED03ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return (float)(uint32_t)(z >> 40) * (1.0f / 16777216.0f);
}

void or_dropout_forward(float *x, int n, float probability,
                        uint64_t seed, uint32_t iter, uint32_t layer)
{
    const float scale = 1. / (1.0 - probability);
    for (int i = 0; i < n; ++i) {
        float r = or_dropout_uniform(seed, iter, layer, (uint32_t)i);
        if (r < probability) x[i] = 0;
        else x[i] *= scale;
    }
}

void or_dropout_backward(float *delta, int n, float probability,
                         uint64_t seed, uint32_t iter, uint32_t layer)
{
    const float scale = 1. / (1.0 - probability);
    for (int i = 0; i < n; ++i) {
        float r = or_dropout_uniform(seed, iter, layer, (uint32_t)i);
        if (r < probability) delta[i] = 0;
        else delta[i] *= scale;
    }
}

/* ------------------------------------------------------------------------ */
/* SGD update: ConvolutionalLayer.c:959-980 -> WeightData.c:56-61
 * (addWeightToUpdates), :45-50 (addUpdatesToWeight), :73-78 (scaleUpdates),
 * BiasData.c:79-94, ScaleData.c:48-73.                                     */
void or_conv_update(int nweights, float *weights, float *weight_updates,
                    int n, float *biases, float *bias_updates,
                    float *scales, float *scale_updates,
                    int batch, float learning_rate, float momentum, float decay)
{
    const float a1 = -decay * batch;
    const float a2 = learning_rate / batch;
    for (int i = 0; i < nweights; i++) weight_updates[i] += a1 * weights[i];
    for (int i = 0; i < nweights; i++) weights[i] += a2 * weight_updates[i];
    for (int i = 0; i < nweights; i++) weight_updates[i] *= momentum;
    for (int i = 0; i < n; i++) biases[i] += a2 * bias_updates[i];
    for (int i = 0; i < n; i++) bias_updates[i] *= momentum;
    if (scales) {
        for (int i = 0; i < n; i++) scales[i] += a2 * scale_updates[i];
        for (int i = 0; i < n; i++) scale_updates[i] *= momentum;
    }
}

/* ------------------------------------------------------------------------ */
/* Weight init: WeightData.c:153-166 (scale*randUniform(-1,1)),
 * DnnUtils.c:196-209 (randUniform over rand(), RAND_MAX >= 65536 branch).  */
void or_rand_seed(unsigned seed) { srand(seed); }

float or_rand_uniform(float min, float max)
{
    if (max < min) {
        float swap = min;
        min = max;
        max = swap;
    }
    return ((float)rand() / RAND_MAX * (max - min)) + min;
}

/* ======================================================================== */
/* Network: NNetwork.c:382-396 (forward), :627-654 (backward), :667-680
 * (updateCPU), :740-758 (train), :762-805 (train + update + return).       */
enum { L_CONV = 0, L_MAXPOOL = 1, L_AVGPOOL = 2, L_DROPOUT = 3, L_SOFTMAX = 4 };

typedef struct {
    int type;
    int batch, inputs, outputs;
    int h, w, c, out_h, out_w, out_c;
    /* conv */
    int n, size, stride, pad, activation, batch_normalize, nweights;
    int stride_y; /* conv and maxpool: height stride (stride is the width one) */
    float *weights, *weight_updates, *biases, *bias_updates;
    float *scales, *scale_updates, *mean, *variance, *rolling_mean, *rolling_variance;
    float *x, *x_norm, *mean_delta, *variance_delta;
    /* maxpool */
    int *indexes;
    /* dropout */
    float probability;
    int shares_prev;
    /* softmax */
    int groups;
    float temperature;
    float *loss;
    float cost;
    float *output, *delta;
    /* NLayer options (NLayer.h:115-121): NNetwork.backward stops before a
     * stopbackward layer and skips an onlyforward one (NNetwork.c:648-651);
     * updateCPU skips train == 0 (NNetwork.c:673-674); the conv update runs
     * at rate * learning_rate_scale (ConvolutionalLayer.c:960)            */
    int stopbackward, onlyforward, train;
    float learning_rate_scale;
} or_layer;

struct or_net {
    int batch, h, w, c;
    int n, cap;
    or_layer *layers;
    float learning_rate, momentum, decay;
    uint64_t dropout_seed;
    uint32_t cur_iteration;
    /* NNetwork.seen / subdivisions (NNetwork.h:32-35); the dropout masks of
     * a minibatch use its index seen/batch taken before seen += batch      */
    uint64_t seen;
    uint32_t dropout_step;
    int subdivisions;
    /* learning-rate policy (NNetwork.h:29-31,39,45-51) */
    int policy, burn_in, step, max_batches, num_steps;
    float power, gamma, scale;
    int *steps;
    float *scales;
    float *workspace;
    size_t workspace_size;
    float *input; /* host copy of the current input (layer 0 reads it) */
    float *truth; /* host copy of the current one-hot truth */
    int has_truth;
};

or_net *or_net_create(int batch, int h, int w, int c)
{
    or_net *net = (or_net *)calloc(1, sizeof(or_net));
    net->batch = batch;
    net->h = h;
    net->w = w;
    net->c = c;
    net->learning_rate = .001f;
    net->momentum = .9f;
    net->decay = .0001f;
    net->dropout_seed = 0x5eed;
    net->subdivisions = 1;
    /* parseNetOption defaults (NetworkFactory.c:763-773,817) */
    net->policy = OR_POLICY_CONSTANT;
    net->power = 4;
    net->gamma = 1;
    net->scale = 1;
    net->step = 1;
    return net;
}

static or_layer *push_layer(or_net *net)
{
    if (net->n == net->cap) {
        net->cap = net->cap ? 2 * net->cap : 16;
        net->layers = (or_layer *)realloc(net->layers, sizeof(or_layer) * net->cap);
    }
    or_layer *l = &net->layers[net->n];
    memset(l, 0, sizeof(*l));
    l->batch = net->batch;
    if (net->n == 0) {
        l->h = net->h;
        l->w = net->w;
        l->c = net->c;
    } else {
        or_layer *p = &net->layers[net->n - 1];
        l->h = p->out_h;
        l->w = p->out_w;
        l->c = p->out_c;
    }
    l->inputs = l->h * l->w * l->c;
    l->train = 1;
    l->learning_rate_scale = 1;
    return l;
}

static float *fzalloc(size_t n) { return (float *)calloc(n ? n : 1, sizeof(float)); }

static int add_conv(or_net *net, int filters, int size, int stride, int stride_y, int pad,
                    int activation, int batch_normalize, int flatten)
{
    or_layer *l = push_layer(net);
    if (flatten) { /* [batch][c][h][w] read as [batch][c*h*w][1][1] */
        l->c = l->c * l->h * l->w;
        l->h = l->w = 1;
    }
    l->type = L_CONV;
    l->n = filters;
    l->size = size;
    l->stride = stride;
    l->stride_y = stride_y;
    l->pad = pad;
    l->activation = activation;
    l->batch_normalize = batch_normalize;
    l->out_h = (l->h + 2 * pad - size) / stride_y + 1;
    l->out_w = (l->w + 2 * pad - size) / stride + 1;
    l->out_c = filters;
    if (l->out_h <= 0 || l->out_w <= 0) return -1;
    l->outputs = l->out_h * l->out_w * l->out_c;
    l->nweights = l->c * filters * size * size;
    size_t bo = (size_t)l->batch * l->outputs;
    l->output = fzalloc(bo);
    l->delta = fzalloc(bo);
    l->weights = fzalloc(l->nweights);
    l->weight_updates = fzalloc(l->nweights);
    l->biases = fzalloc(filters);
    l->bias_updates = fzalloc(filters);
    /* WeightData.c:153-166: scale = sqrt(2/(k*k*c)) */
    float scale = sqrt(2. / (size * size * l->c));
    for (int i = 0; i < l->nweights; ++i) l->weights[i] = scale * or_rand_uniform(-1, 1);
    if (batch_normalize) {
        l->scales = fzalloc(filters);
        for (int i = 0; i < filters; ++i) l->scales[i] = 1;
        l->scale_updates = fzalloc(filters);
        l->mean = fzalloc(filters);
        l->variance = fzalloc(filters);
        l->rolling_mean = fzalloc(filters);
        l->rolling_variance = fzalloc(filters);
        l->mean_delta = fzalloc(filters);
        l->variance_delta = fzalloc(filters);
        l->x = fzalloc(bo);
        l->x_norm = fzalloc(bo);
    }
    return net->n++;
}

int or_net_add_conv(or_net *net, int filters, int size, int stride, int pad,
                    int activation, int batch_normalize)
{
    return add_conv(net, filters, size, stride, stride, pad, activation, batch_normalize, 0);
}

int or_net_add_conv_xy(or_net *net, int filters, int size, int stride_x, int stride_y, int pad,
                       int activation, int batch_normalize)
{
    return add_conv(net, filters, size, stride_x, stride_y, pad, activation, batch_normalize, 0);
}

/* A fully connected layer (darknet's [connected]; the reference builds none,
 * NetworkFactory.c:615-654): the previous output flattened to c*h*w
 * features, then the 1x1 convolution path of this file -- out_i = W x_i
 * (Gemm.c:53-66), bias or batch-norm, activation -- with init
 * sqrt(2/inputs)*randUniform(-1,1) (WeightData.c:153-166 with k = 1).      */
int or_net_add_connected(or_net *net, int outputs, int activation, int batch_normalize)
{
    return add_conv(net, outputs, 1, 1, 1, 0, activation, batch_normalize, 1);
}

int or_net_add_maxpool(or_net *net, int size, int stride, int padding)
{
    return or_net_add_maxpool_xy(net, size, stride, stride, padding);
}

int or_net_add_maxpool_xy(or_net *net, int size, int stride_x, int stride_y, int padding)
{
    or_layer *l = push_layer(net);
    l->type = L_MAXPOOL;
    l->size = size;
    l->stride = stride_x;
    l->stride_y = stride_y;
    l->pad = padding;
    l->out_h = or_maxpool_out(l->h, size, stride_y, padding);
    l->out_w = or_maxpool_out(l->w, size, stride_x, padding);
    l->out_c = l->c;
    if (l->out_h <= 0 || l->out_w <= 0) return -1;
    l->outputs = l->out_h * l->out_w * l->out_c;
    size_t bo = (size_t)l->batch * l->outputs;
    l->output = fzalloc(bo);
    l->delta = fzalloc(bo);
    l->indexes = (int *)calloc(bo, sizeof(int));
    return net->n++;
}

int or_net_add_avgpool(or_net *net)
{
    or_layer *l = push_layer(net);
    l->type = L_AVGPOOL;
    l->out_h = l->out_w = 1;
    l->out_c = l->c;
    l->outputs = l->c;
    l->output = fzalloc((size_t)l->batch * l->outputs);
    l->delta = fzalloc((size_t)l->batch * l->outputs);
    return net->n++;
}

int or_net_add_dropout(or_net *net, float probability)
{
    if (net->n == 0) return -1;
    or_layer *l = push_layer(net);
    or_layer *p = &net->layers[net->n - 1];
    l->type = L_DROPOUT;
    l->probability = probability;
    l->out_h = l->h;
    l->out_w = l->w;
    l->out_c = l->c;
    l->outputs = l->inputs;
    /* NetworkFactory.c:644-650: share the previous layer's output and delta */
    l->output = p->output;
    l->delta = p->delta;
    l->shares_prev = 1;
    return net->n++;
}

int or_net_add_softmax(or_net *net, int groups, float temperature)
{
    or_layer *l = push_layer(net);
    l->type = L_SOFTMAX;
    l->groups = groups;
    l->temperature = temperature;
    l->out_h = l->h;
    l->out_w = l->w;
    l->out_c = l->c;
    l->outputs = l->inputs;
    size_t bo = (size_t)l->batch * l->outputs;
    l->output = fzalloc(bo);
    l->delta = fzalloc(bo);
    l->loss = fzalloc(bo);
    return net->n++;
}

void or_net_set_hyper(or_net *net, float learning_rate, float momentum, float decay)
{
    net->learning_rate = learning_rate;
    net->momentum = momentum;
    net->decay = decay;
}

void or_net_set_dropout_seed(or_net *net, uint64_t seed) { net->dropout_seed = seed; }

void or_net_set_subdivisions(or_net *net, int subdivisions)
{
    net->subdivisions = subdivisions > 0 ? subdivisions : 1;
}

void or_net_set_policy(or_net *net, int policy, int burn_in, float power, float gamma,
                       float scale, int step, int max_batches, int num_steps, const int *steps,
                       const float *scales)
{
    net->policy = policy;
    net->burn_in = burn_in;
    net->power = power;
    net->gamma = gamma;
    net->scale = scale;
    net->step = step;
    net->max_batches = max_batches;
    free(net->steps);
    free(net->scales);
    net->steps = NULL;
    net->scales = NULL;
    net->num_steps = num_steps > 0 ? num_steps : 0;
    if (net->num_steps) {
        net->steps = (int *)malloc(sizeof(int) * net->num_steps);
        net->scales = (float *)malloc(sizeof(float) * net->num_steps);
        memcpy(net->steps, steps, sizeof(int) * net->num_steps);
        memcpy(net->scales, scales, sizeof(float) * net->num_steps);
    }
}

/* NNetwork.getCurrentRate (NNetwork.c:215-246) with the reference's types:
 * batch_num is size_t (getCurrentBatch, NNetwork.c:154-157), so in the
 * sigmoid policy batch_num - step wraps around below step (the rate is
 * then 0 for gamma > 0); burn_in and steps[i] compare as size_t.  The
 * random policy draws randUniform(0,1) from rand().                     */
float or_lr_rate(int policy, float learning_rate, uint64_t batch_num64, int burn_in, float power,
                 float gamma, float scale, int step, int max_batches, int num_steps,
                 const int *steps, const float *scales)
{
    const size_t batch_num = (size_t)batch_num64;
    if (batch_num < (size_t)burn_in)
        return learning_rate * pow((float)batch_num / burn_in, power);
    switch (policy) {
    case OR_POLICY_CONSTANT: return learning_rate;
    case OR_POLICY_STEP: return learning_rate * pow(scale, batch_num / (size_t)step);
    case OR_POLICY_STEPS: {
        float rate = learning_rate;
        for (int i = 0; i < num_steps; ++i) {
            if ((size_t)steps[i] > batch_num) return rate;
            rate *= scales[i];
        }
        return rate;
    }
    case OR_POLICY_EXP: return learning_rate * pow(gamma, (int)batch_num);
    case OR_POLICY_POLY: return learning_rate * pow(1 - (float)batch_num / max_batches, power);
    case OR_POLICY_RANDOM: return learning_rate * pow(or_rand_uniform(0, 1), power);
    case OR_POLICY_SIG:
        return learning_rate * (1. / (1. + exp(gamma * (float)(batch_num - (size_t)step))));
    default: return learning_rate;
    }
}

float or_net_rate(or_net *net)
{
    const uint64_t batch_num = net->seen / ((uint64_t)net->batch * net->subdivisions);
    return or_lr_rate(net->policy, net->learning_rate, batch_num, net->burn_in, net->power,
                      net->gamma, net->scale, net->step, net->max_batches, net->num_steps,
                      net->steps, net->scales);
}

void or_net_set_layer_options(or_net *net, int i, int stopbackward, int onlyforward,
                              float learning_rate_scale)
{
    or_layer *l = &net->layers[i];
    l->stopbackward = stopbackward;
    l->onlyforward = onlyforward;
    l->learning_rate_scale = learning_rate_scale;
}

int or_net_finalize(or_net *net)
{
    /* NetworkFactory.c:881-893, 981-991: every layer below the last layer
     * whose stopbackward is exactly 1 (atoi(value) == 1 at :889-890) runs
     * forward only and is not updated; the backward loop stops at any
     * nonzero value (NNetwork.c:648) */
    int last_stop = -1;
    for (int i = 0; i < net->n; ++i)
        if (net->layers[i].stopbackward == 1) last_stop = i;
    for (int k = 0; k < last_stop; ++k) {
        net->layers[k].onlyforward = 1;
        net->layers[k].train = 0;
    }
    size_t ws = 0;
    for (int i = 0; i < net->n; ++i) {
        or_layer *l = &net->layers[i];
        if (l->type != L_CONV) continue;
        or_conv_shape s = {l->batch, l->c, l->h, l->w, l->n, l->size, l->stride, l->pad,
                           l->stride_y};
        size_t need = or_conv_workspace_floats(&s);
        if (need > ws) ws = need;
    }
    net->workspace_size = ws;
    net->workspace = fzalloc(ws);
    net->input = fzalloc((size_t)net->batch * net->h * net->w * net->c);
    net->truth = fzalloc((size_t)net->batch * net->layers[net->n - 1].outputs);
    return 0;
}

void or_net_free(or_net *net)
{
    if (!net) return;
    for (int i = 0; i < net->n; ++i) {
        or_layer *l = &net->layers[i];
        if (!l->shares_prev) {
            free(l->output);
            free(l->delta);
        }
        free(l->weights); free(l->weight_updates); free(l->biases); free(l->bias_updates);
        free(l->scales); free(l->scale_updates); free(l->mean); free(l->variance);
        free(l->rolling_mean); free(l->rolling_variance); free(l->x); free(l->x_norm);
        free(l->mean_delta); free(l->variance_delta); free(l->indexes); free(l->loss);
    }
    free(net->layers);
    free(net->workspace);
    free(net->input);
    free(net->truth);
    free(net->steps);
    free(net->scales);
    free(net);
}

typedef struct {
    const float *truth;
    float *input;
    float *delta;
    int train;
    int index;
} or_state;

static void conv_forward(or_net *net, or_layer *l, or_state st)
{
    or_conv_shape s = {l->batch, l->c, l->h, l->w, l->n, l->size, l->stride, l->pad,
                       l->stride_y};
    const int spatial = l->out_h * l->out_w;
    or_conv_forward(&s, st.input, l->weights, l->output, net->workspace);
    if (l->batch_normalize && !st.train) {
        /* forwardNormCPU, NLayer.c:141-162 (inference branch): normalizeByRoll
         * copies the pre-BN tensor to x, then normalizes with the rolling
         * statistics (NormData.c:291-326) */
        memcpy(l->x, l->output, sizeof(float) * (size_t)l->batch * l->outputs);
        or_bn_normalize_roll(l->output, l->batch, l->n, spatial, l->rolling_mean,
                             l->rolling_variance, l->scales, l->biases);
    } else if (l->batch_normalize) {
        /* forwardNormCPU, NLayer.c:141-162 (train branch) */
        or_bn_mean_var(l->output, l->batch, l->n, spatial, l->mean, l->variance);
        or_bn_roll(l->n, l->mean, l->variance, l->rolling_mean, l->rolling_variance);
        if (or_bn_normalize(l->output, l->batch, l->n, spatial, l->mean, l->variance,
                            l->scales, l->biases, l->x, l->x_norm))
            fprintf(stderr, "oracle: NaN in batch-norm normalize (layer %d)\n", st.index);
    } else {
        or_add_bias(l->output, l->biases, l->batch, l->n, spatial);
    }
    or_activate(l->output, l->batch * l->outputs, l->activation);
}

static void conv_backward(or_net *net, or_layer *l, or_state st)
{
    or_conv_shape s = {l->batch, l->c, l->h, l->w, l->n, l->size, l->stride, l->pad,
                       l->stride_y};
    const int spatial = l->out_h * l->out_w;
    or_gradient(l->output, l->batch * l->outputs, l->activation, l->delta);
    if (l->batch_normalize)
        or_bn_backward(l->delta, l->batch, l->n, spatial, l->x, l->x_norm, l->mean,
                       l->variance, l->scales, l->scale_updates, l->mean_delta,
                       l->variance_delta);
    else
        or_bias_grad(l->bias_updates, l->delta, l->batch, l->n, spatial);
    or_conv_backward(&s, st.input, l->delta, l->weights, l->weight_updates, st.delta,
                     net->workspace);
}

static void layer_forward(or_net *net, or_layer *l, or_state st)
{
    switch (l->type) {
    case L_CONV: conv_forward(net, l, st); break;
    case L_MAXPOOL:
        or_maxpool_forward_xy(st.input, l->batch, l->c, l->h, l->w, l->size, l->stride,
                              l->stride_y, l->pad, l->output, l->indexes);
        break;
    case L_AVGPOOL:
        or_avgpool_forward(st.input, l->batch, l->c, l->h * l->w, l->output);
        break;
    case L_DROPOUT:
        if (st.train)
            or_dropout_forward(st.input, l->batch * l->inputs, l->probability,
                               net->dropout_seed, net->dropout_step, (uint32_t)st.index);
        break;
    case L_SOFTMAX:
        l->cost = or_softmax_xent_forward(st.input, l->batch, l->inputs, l->groups,
                                          l->temperature, st.truth, l->output, l->delta,
                                          l->loss);
        break;
    }
}

static void layer_backward(or_net *net, or_layer *l, or_state st)
{
    switch (l->type) {
    case L_CONV: conv_backward(net, l, st); break;
    case L_MAXPOOL:
        if (st.delta)
            or_maxpool_backward(l->delta, l->indexes, l->batch * l->outputs, st.delta);
        break;
    case L_AVGPOOL:
        if (st.delta)
            or_avgpool_backward(l->delta, l->batch, l->c, l->h * l->w, st.delta);
        break;
    case L_DROPOUT:
        if (st.delta)
            or_dropout_backward(st.delta, l->batch * l->inputs, l->probability,
                                net->dropout_seed, net->dropout_step, (uint32_t)st.index);
        break;
    case L_SOFTMAX:
        if (st.delta) or_softmax_backward(l->delta, l->batch * l->inputs, st.delta);
        break;
    }
}

void or_net_load(or_net *net, const float *input, const float *truth)
{
    size_t in_n = (size_t)net->batch * net->h * net->w * net->c;
    memcpy(net->input, input, in_n * sizeof(float));
    if (truth) {
        const or_layer *last = &net->layers[net->n - 1];
        size_t tn = (size_t)net->batch * last->outputs;
        memcpy(net->truth, truth, tn * sizeof(float));
        net->has_truth = 1;
    } else {
        net->has_truth = 0;
    }
}

static or_state fwd_state(or_net *net, int i, int train)
{
    or_state st = {net->has_truth ? net->truth : NULL, net->input, NULL, train, i};
    if (i > 0) st.input = net->layers[i - 1].output;
    return st;
}

static or_state bwd_state(or_net *net, int i)
{
    or_state st = {net->has_truth ? net->truth : NULL, net->input, NULL, 1, i};
    if (i > 0) {
        st.input = net->layers[i - 1].output;
        st.delta = net->layers[i - 1].delta;
    }
    return st;
}

/* One layer of NNetwork.forward (NNetwork.c:385-395): zero its delta, run. */
void or_net_layer_forward(or_net *net, int i, int train)
{
    or_layer *l = &net->layers[i];
    if (train && l->delta) memset(l->delta, 0, sizeof(float) * (size_t)l->batch * l->outputs);
    layer_forward(net, l, fwd_state(net, i, train));
}

/* One layer of NNetwork.backward (NNetwork.c:631-652). */
void or_net_layer_backward(or_net *net, int i)
{
    layer_backward(net, &net->layers[i], bwd_state(net, i));
}

float or_net_cost(or_net *net)
{
    /* getNetworkCost (NNetwork.c:611-624) then sum/(subdivisions*batch) */
    float sum = 0;
    int count = 0;
    for (int i = 0; i < net->n; ++i)
        if (net->layers[i].type == L_SOFTMAX) {
            sum += net->layers[i].cost;
            ++count;
        }
    float cost = count ? sum / count : 0;
    return cost / net->batch;
}

/* NNetwork.train(input, truth) (NNetwork.c:740-758): seen += batch, then
 * forward and backward; returns the cost / batch.                        */
float or_net_forward_backward(or_net *net, const float *input, const float *truth)
{
    net->dropout_step = (uint32_t)(net->seen / (uint64_t)net->batch);
    net->seen += (uint64_t)net->batch;
    or_net_load(net, input, truth);
    for (int i = 0; i < net->n; ++i) or_net_layer_forward(net, i, 1);
    for (int i = net->n - 1; i >= 0; --i) {
        if (net->layers[i].stopbackward) break;
        if (net->layers[i].onlyforward) continue;
        or_net_layer_backward(net, i);
    }
    return or_net_cost(net);
}

/* cur_iteration += 1, then updateCPU (NNetwork.c:667-680, 788-789): every
 * conv layer with update batch = batch * subdivisions and the policy's rate */
void or_net_update(or_net *net)
{
    net->cur_iteration += 1;
    const int update_batch = net->batch * net->subdivisions;
    const float rate = or_net_rate(net);
    for (int i = 0; i < net->n; ++i) {
        or_layer *l = &net->layers[i];
        if (l->type != L_CONV || !l->train) continue;
        or_conv_update(l->nweights, l->weights, l->weight_updates, l->n, l->biases,
                       l->bias_updates, l->scales, l->scale_updates, update_batch,
                       rate * l->learning_rate_scale, net->momentum, net->decay);
    }
}

/* NNetwork.predict (NNetwork.c:411-422): forward with train = 0 and no
 * truth, then the output of the last non-cost layer (NNetwork.c:400-407),
 * batch x outputs floats, is copied to `output`.                          */
void or_net_predict(or_net *net, const float *input, float *output)
{
    or_net_load(net, input, NULL);
    for (int i = 0; i < net->n; ++i) layer_forward(net, &net->layers[i], fwd_state(net, i, 0));
    const or_layer *last = &net->layers[net->n - 1];
    memcpy(output, last->output, sizeof(float) * (size_t)last->batch * last->outputs);
}

/* NNetwork.fuseConvBatchnorm (NNetwork.c:272-288), conv layers: fold each
 * BN conv layer (or_conv_bn_fold) and turn it into a plain conv with bias
 * (batch_normalize = 0; the BN arrays are no longer read).                 */
void or_net_fuse_conv_batchnorm(or_net *net)
{
    for (int i = 0; i < net->n; ++i) {
        or_layer *l = &net->layers[i];
        if (l->type != L_CONV || !l->batch_normalize) continue;
        or_conv_bn_fold(l->n, l->nweights / l->n, l->weights, l->biases, l->scales,
                        l->rolling_mean, l->rolling_variance);
        l->batch_normalize = 0;
    }
}

/* One minibatch of NNetwork.train(ImageData) (NNetwork.c:762-805): the
 * update runs after every subdivisions-th minibatch, when the gradient sums
 * hold the whole batch * subdivisions images.                             */
float or_net_train(or_net *net, const float *input, const float *truth)
{
    float loss = or_net_forward_backward(net, input, truth);
    if ((net->seen / (uint64_t)net->batch) % (uint64_t)net->subdivisions == 0) or_net_update(net);
    return loss;
}

uint64_t or_net_seen(const or_net *net) { return net->seen; }
int or_net_iteration(const or_net *net) { return (int)net->cur_iteration; }

int or_net_n_layers(const or_net *net) { return net->n; }

void *or_net_buffer(or_net *net, int li, int which, size_t *count)
{
    *count = 0;
    if (li < 0 || li >= net->n) return NULL;
    or_layer *l = &net->layers[li];
    size_t bo = (size_t)l->batch * l->outputs;
    switch (which) {
    case 0: *count = bo; return l->output;
    case 1: *count = bo; return l->delta;
    case 2: *count = l->weights ? (size_t)l->nweights : 0; return l->weights;
    case 3: *count = l->weight_updates ? (size_t)l->nweights : 0; return l->weight_updates;
    case 4: *count = l->biases ? (size_t)l->n : 0; return l->biases;
    case 5: *count = l->bias_updates ? (size_t)l->n : 0; return l->bias_updates;
    case 6: *count = l->scales ? (size_t)l->n : 0; return l->scales;
    case 7: *count = l->scale_updates ? (size_t)l->n : 0; return l->scale_updates;
    case 8: *count = l->rolling_mean ? (size_t)l->n : 0; return l->rolling_mean;
    case 9: *count = l->rolling_variance ? (size_t)l->n : 0; return l->rolling_variance;
    case 10: *count = l->mean ? (size_t)l->n : 0; return l->mean;
    case 11: *count = l->variance ? (size_t)l->n : 0; return l->variance;
    case 12: *count = l->x ? bo : 0; return l->x;
    case 13: *count = l->x_norm ? bo : 0; return l->x_norm;
    case 14: *count = l->indexes ? bo : 0; return l->indexes;
    case 15: *count = l->loss ? bo : 0; return l->loss;
    }
    return NULL;
}

void or_net_layer_info(const or_net *net, int li, int *info)
{
    memset(info, 0, sizeof(int) * 8);
    if (li < 0 || li >= net->n) return;
    const or_layer *l = &net->layers[li];
    info[0] = l->type;
    info[1] = l->out_c;
    info[2] = l->out_h;
    info[3] = l->out_w;
    info[4] = l->c;
    info[5] = l->h;
    info[6] = l->w;
    info[7] = l->batch;
}
