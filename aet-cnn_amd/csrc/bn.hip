// Batch-norm in training mode with the reference CPU path's arithmetic.
//
// Forward  = forwardNormCPU (NLayer.c:141-162):
//   NormData.calcVarianceAndMean  NormData.c:141-186  unbiased, sum-of-squares
//   scalAxpyRollMeanAndRollVariance NormData.c:224-229 rolling .9/.1
//   NormData.normalize            NormData.c:244-282  inv = 1/(sqrt(var)+1e-6)
// Backward = backwardNormCPU (NLayer.c:246-278):
//   ScaleData.backwardScale ScaleData.c:76-107, NData.scale NData.c:238-248,
//   DeltaData.calcMean/calcVariance/normalize DeltaData.c:23-80 (eps 1e-5,
//   double sub-expressions); no beta gradient.
//
// Each direction is a per-channel reduction pass (grid = channels x batch
// chunks, double accumulation, one partial per block, no atomics), a one-
// thread-per-channel finalize that combines the partials in a fixed order,
// and one coalesced elementwise pass (float4 when H*W % 4 == 0).  The
// activation that follows BN in a conv layer can be fused into the forward
// apply and its gradient into both backward passes; the gradient's sign is
// taken from the recomputed BN output (same float ops as the forward), so
// the activated tensor does not have to be re-read.
#include "common.hpp"

namespace ach {

constexpr int BN_NT = 256;

static int bn_chunks(int batch, int c)
{
    int nch = (2048 + c - 1) / c;
    if (nch > batch) nch = batch;
    if (nch < 1) nch = 1;
    return nch;
}

template <int NV>
__device__ __forceinline__ double block_sum(double v, double *sh)
{
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) sh[w] = v;
    __syncthreads();
    double t = 0;
    if (threadIdx.x == 0)
        for (int i = 0; i < NV; ++i) t += sh[i];
    return t;  // valid in thread 0
}

// ---- forward statistics: partial[ch][c] = {sum x, sum x^2} -----------------
__global__ void __launch_bounds__(BN_NT) k_bn_stats(const float *__restrict__ x, int batch,
                                                    int C, int HW, int per,
                                                    double *__restrict__ part)
{
    __shared__ double sh[BN_NT / 64];
    const int c = blockIdx.x, ch = blockIdx.y;
    const int b0 = ch * per, b1 = min(batch, b0 + per);
    double s1 = 0, s2 = 0;
    if ((HW & 3) == 0) {
        const int hw4 = HW >> 2;
        const int tot = (b1 - b0) * hw4;
        for (int i = threadIdx.x; i < tot; i += BN_NT) {
            const int bb = b0 + i / hw4, q = i - (i / hw4) * hw4;
            const float4 v = reinterpret_cast<const float4 *>(x + ((size_t)bb * C + c) * HW)[q];
            s1 += (double)v.x + (double)v.y + (double)v.z + (double)v.w;
            s2 += (double)(v.x * v.x) + (double)(v.y * v.y) + (double)(v.z * v.z) +
                  (double)(v.w * v.w);
        }
    } else {
        const int tot = (b1 - b0) * HW;
        for (int i = threadIdx.x; i < tot; i += BN_NT) {
            const int bb = b0 + i / HW, q = i - (i / HW) * HW;
            const float v = x[((size_t)bb * C + c) * HW + q];
            s1 += v;
            s2 += (double)(v * v);
        }
    }
    const double t1 = block_sum<BN_NT / 64>(s1, sh);
    const double t2 = block_sum<BN_NT / 64>(s2, sh);
    if (threadIdx.x == 0) {
        part[((size_t)ch * C + c) * 2 + 0] = t1;
        part[((size_t)ch * C + c) * 2 + 1] = t2;
    }
}

// ---- forward finalize: mean, unbiased variance, rolling stats, inv --------
__global__ void k_bn_finalize(const double *__restrict__ part, int nch, int C, int batch,
                              int HW, float *__restrict__ mean, float *__restrict__ variance,
                              float *__restrict__ rmean, float *__restrict__ rvar,
                              float *__restrict__ inv)
{
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= C) return;
    double S1 = 0, S2 = 0;
    for (int ch = 0; ch < nch; ++ch) {
        S1 += part[((size_t)ch * C + c) * 2 + 0];
        S2 += part[((size_t)ch * C + c) * 2 + 1];
    }
    // NormData.c:170-185 in float: mean = (sum x) * (1/N);
    // var = (t1 + t2*mean + mean*mean*batch*spatial) * (1/(N-1)), t2 = sum(-2x)
    const int N = batch * HW;
    const float scale = (float)(1. / N);
    const float m = (float)S1 * scale;
    const float t1 = (float)S2, t2 = (float)(-2.0 * S1);
    float mm = m * m;
    mm = mm * (float)batch;
    mm = mm * (float)HW;
    float v = t1 + t2 * m + mm;
    v *= (float)(1. / (N - 1));
    mean[c] = m;
    variance[c] = v;
    if (rmean) {
        const float keep = .9f, take = .1f;
        rmean[c] = rmean[c] * keep;
        rmean[c] += take * m;
        rvar[c] = rvar[c] * keep;
        rvar[c] += take * v;
    }
    inv[c] = (float)(1.0 / (sqrt((double)v) + (double)1e-6f));
}

__global__ void k_bn_inv(const float *__restrict__ variance, int C, float *__restrict__ inv)
{
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c < C) inv[c] = (float)(1.0 / (sqrt((double)variance[c]) + (double)1e-6f));
}

// ---- forward apply ----------------------------------------------------------
// src: pre-BN tensor; xcopy (optional) gets a copy; xnorm (optional);
// out = act(xnorm*scale + bias).
__global__ void __launch_bounds__(256) k_bn_apply(const float *src, float *xcopy,
                                                  float *xnorm, float *out,
                                                  size_t total, int C, int HW,
                                                  const float *__restrict__ mean,
                                                  const float *__restrict__ inv,
                                                  const float *__restrict__ scales,
                                                  const float *__restrict__ biases, int act)
{
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    if ((HW & 3) == 0) {
        const size_t tot4 = total >> 2;
        const int hw4 = HW >> 2;
        for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < tot4; i += stride) {
            const int c = (int)((i / hw4) % C);
            const float mu = mean[c], iv = inv[c], s = scales[c], bb = biases[c];
            float4 v = reinterpret_cast<const float4 *>(src)[i];
            if (xcopy) reinterpret_cast<float4 *>(xcopy)[i] = v;
            float4 n;
            n.x = (v.x - mu) * iv; n.y = (v.y - mu) * iv;
            n.z = (v.z - mu) * iv; n.w = (v.w - mu) * iv;
            if (xnorm) reinterpret_cast<float4 *>(xnorm)[i] = n;
            float4 o;
            o.x = act_forward(__fmaf_rn(n.x, s, bb), act);
            o.y = act_forward(__fmaf_rn(n.y, s, bb), act);
            o.z = act_forward(__fmaf_rn(n.z, s, bb), act);
            o.w = act_forward(__fmaf_rn(n.w, s, bb), act);
            reinterpret_cast<float4 *>(out)[i] = o;
        }
    } else {
        for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += stride) {
            const int c = (int)((i / HW) % C);
            const float v = src[i];
            if (xcopy) xcopy[i] = v;
            const float n = (v - mean[c]) * inv[c];
            if (xnorm) xnorm[i] = n;
            out[i] = act_forward(__fmaf_rn(n, scales[c], biases[c]), act);
        }
    }
}

// ---- backward ---------------------------------------------------------------
// Activation gradient evaluated from the recomputed BN output z: y>0 <=> z>0
// for leaky and relu, so f'(y) == f'(z-derived) bit for bit.
__device__ __forceinline__ float bwd_grad(float d, float xv, float mu, float iv, float s,
                                          float bb, int act)
{
    if (act == ACH_LEAKY || act == ACH_RELU) {
        const float z = __fmaf_rn((xv - mu) * iv, s, bb);
        const float y = act_forward(z, act);
        d *= act_gradient(y, act);
    }
    return d;
}

// partial[ch][c] = {sum g*xn, sum g*s, sum (g*s)*(x-mean)}
__global__ void __launch_bounds__(BN_NT) k_bn_bwd_reduce(
    const float *__restrict__ delta, const float *__restrict__ x,
    const float *__restrict__ xnorm, int batch, int C, int HW, int per,
    const float *__restrict__ mean, const float *__restrict__ inv,
    const float *__restrict__ scales, const float *__restrict__ biases, int act,
    double *__restrict__ part)
{
    __shared__ double sh[BN_NT / 64];
    const int c = blockIdx.x, ch = blockIdx.y;
    const int b0 = ch * per, b1 = min(batch, b0 + per);
    const float mu = mean[c], iv = inv[c], s = scales[c], bb = biases ? biases[c] : 0.f;
    double g1 = 0, g2 = 0, g3 = 0;
    const int tot = (b1 - b0) * HW;
    for (int i = threadIdx.x; i < tot; i += BN_NT) {
        const int b = b0 + i / HW, q = i - (i / HW) * HW;
        const size_t idx = ((size_t)b * C + c) * HW + q;
        const float xv = x[idx];
        const float g = bwd_grad(delta[idx], xv, mu, iv, s, bb, act);
        const float xn = xnorm ? xnorm[idx] : (xv - mu) * iv;
        const float gs = g * s;
        g1 += (double)(g * xn);
        g2 += (double)gs;
        g3 += (double)(gs * (xv - mu));
    }
    const double t1 = block_sum<BN_NT / 64>(g1, sh);
    const double t2 = block_sum<BN_NT / 64>(g2, sh);
    const double t3 = block_sum<BN_NT / 64>(g3, sh);
    if (threadIdx.x == 0) {
        double *p = part + ((size_t)ch * C + c) * 3;
        p[0] = t1; p[1] = t2; p[2] = t3;
    }
}

// coef[c] = {1/sqrt(var+1e-5), 2*variance_delta/N, mean_delta/N}
__global__ void k_bn_bwd_finalize(const double *__restrict__ part, int nch, int C, int N,
                                  const float *__restrict__ variance,
                                  float *__restrict__ scale_updates,
                                  float *__restrict__ mean_delta,
                                  float *__restrict__ variance_delta,
                                  double *__restrict__ coef)
{
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= C) return;
    double G1 = 0, G2 = 0, G3 = 0;
    for (int ch = 0; ch < nch; ++ch) {
        const double *p = part + ((size_t)ch * C + c) * 3;
        G1 += p[0]; G2 += p[1]; G3 += p[2];
    }
    scale_updates[c] += (float)G1;
    const float ve = variance[c] + 1e-5f;
    // DeltaData.c:36  mean *= (-1./sqrt(var + 1e-5f))
    const float md = (float)((double)(float)G2 * (-1. / sqrt((double)ve)));
    // DeltaData.c:56  variance *= -.5 * pow(var + 1e-5f, -1.5f)
    const float vd = (float)((double)(float)G3 * (-.5 * pow((double)ve, (double)(-1.5f))));
    if (mean_delta) mean_delta[c] = md;
    if (variance_delta) variance_delta[c] = vd;
    coef[(size_t)c * 3 + 0] = 1. / sqrt((double)ve);
    coef[(size_t)c * 3 + 1] = (double)vd * 2. / (double)N;
    coef[(size_t)c * 3 + 2] = (double)(md / (float)N);
}

// DeltaData.c:64-80: d = d*1/sqrt(v+1e-5) + vd*2*(x-mu)/N + md/N (double)
__global__ void __launch_bounds__(256) k_bn_bwd_apply(
    float *__restrict__ delta, const float *__restrict__ x, size_t total, int C, int HW,
    const float *__restrict__ mean, const float *__restrict__ inv,
    const float *__restrict__ scales, const float *__restrict__ biases, int act,
    const double *__restrict__ coef)
{
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += stride) {
        const int c = (int)((i / HW) % C);
        const float mu = mean[c], s = scales[c];
        const float xv = x[i];
        const float g = bwd_grad(delta[i], xv, mu, inv[c], s, biases ? biases[c] : 0.f, act);
        const float gs = g * s;
        const double *k = coef + (size_t)c * 3;
        delta[i] = (float)((double)gs * k[0] + k[1] * (double)(xv - mu) + k[2]);
    }
}

struct BnWs {
    double *part;
    double *coef;
    float *inv;
};

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

static size_t bn_ws_bytes(int batch, int c)
{
    const int nch = bn_chunks(batch, c);
    return align256((size_t)nch * c * 3 * sizeof(double)) + align256((size_t)c * 3 * sizeof(double)) +
           align256((size_t)c * sizeof(float));
}

static BnWs bn_ws(void *ws, int batch, int c)
{
    const int nch = bn_chunks(batch, c);
    char *p = (char *)ws;
    BnWs w;
    w.part = (double *)p;
    p += align256((size_t)nch * c * 3 * sizeof(double));
    w.coef = (double *)p;
    p += align256((size_t)c * 3 * sizeof(double));
    w.inv = (float *)p;
    return w;
}

static bool bn_args_ok(int batch, int c, int spatial)
{
    return batch > 0 && c > 0 && spatial > 0 && (double)batch * c * spatial < 4.0e18 &&
           (double)batch * spatial > 1.0;
}

static int bn_fwd(const float *src, float *xcopy, float *xnorm, float *out, int batch, int C,
                  int HW, const float *scales, const float *biases, float *mean,
                  float *variance, float *rmean, float *rvar, int act, void *ws,
                  size_t ws_bytes, hipStream_t st)
{
    if (!bn_args_ok(batch, C, HW) || !src || !out || !scales || !biases || !mean || !variance)
        return ACH_EINVAL;
    if ((rmean == nullptr) != (rvar == nullptr)) return ACH_EINVAL;
    if (!ws || ws_bytes < bn_ws_bytes(batch, C)) return ACH_EWORKSPACE;
    const BnWs w = bn_ws(ws, batch, C);
    const int nch = bn_chunks(batch, C);
    const int per = (batch + nch - 1) / nch;
    const int nch_eff = (batch + per - 1) / per;
    hipLaunchKernelGGL(k_bn_stats, dim3(C, nch_eff), dim3(BN_NT), 0, st, src, batch, C, HW, per,
                       w.part);
    int rc = check_launch();
    if (rc) return rc;
    hipLaunchKernelGGL(k_bn_finalize, dim3((C + 63) / 64), dim3(64), 0, st, w.part, nch_eff, C,
                       batch, HW, mean, variance, rmean, rvar, w.inv);
    rc = check_launch();
    if (rc) return rc;
    const size_t total = (size_t)batch * C * HW;
    const size_t work = (HW & 3) == 0 ? total / 4 : total;
    hipLaunchKernelGGL(k_bn_apply, dim3(grid_for(work, 256, 256u * 32u)), dim3(256), 0, st, src,
                       xcopy, xnorm, out, total, C, HW, mean, w.inv, scales, biases, act);
    return check_launch();
}

}  // namespace ach

using namespace ach;

extern "C" {

size_t ach_bn_workspace(int batch, int c, int)
{
    if (batch <= 0 || c <= 0) return 0;
    return bn_ws_bytes(batch, c);
}

int ach_bn_train_fwd(float *out, int batch, int c, int spatial, const float *scales,
                     const float *biases, float *mean, float *variance, float *rolling_mean,
                     float *rolling_variance, float *x, float *x_norm, int activation,
                     void *ws, size_t ws_bytes, ach_stream_t stream)
{
    if (!x || x == out) return ACH_EINVAL;
    return bn_fwd(out, x, x_norm, out, batch, c, spatial, scales, biases, mean, variance,
                  rolling_mean, rolling_variance, activation, ws, ws_bytes, as_stream(stream));
}

int ach_bn_train_fwd_from_x(const float *x, float *out, int batch, int c, int spatial,
                            const float *scales, const float *biases, float *mean,
                            float *variance, float *rolling_mean, float *rolling_variance,
                            int activation, void *ws, size_t ws_bytes, ach_stream_t stream)
{
    if (!x || x == out) return ACH_EINVAL;
    return bn_fwd(x, nullptr, nullptr, out, batch, c, spatial, scales, biases, mean, variance,
                  rolling_mean, rolling_variance, activation, ws, ws_bytes, as_stream(stream));
}

int ach_bn_bwd(float *delta, int batch, int C, int HW, const float *x, const float *x_norm,
               const float *mean, const float *variance, const float *scales,
               const float *biases, float *scale_updates, float *mean_delta,
               float *variance_delta, int activation, void *ws, size_t ws_bytes,
               ach_stream_t stream)
{
    if (!bn_args_ok(batch, C, HW) || !delta || !x || !mean || !variance || !scales ||
        !scale_updates)
        return ACH_EINVAL;
    const bool fused = activation == ACH_LEAKY || activation == ACH_RELU;
    if (fused && !biases) return ACH_EINVAL;
    if (!fused && activation != ACH_LINEAR) return ACH_EUNSUPPORTED;
    if (!ws || ws_bytes < bn_ws_bytes(batch, C)) return ACH_EWORKSPACE;
    hipStream_t st = as_stream(stream);
    const BnWs w = bn_ws(ws, batch, C);
    const int nch = bn_chunks(batch, C);
    const int per = (batch + nch - 1) / nch;
    const int nch_eff = (batch + per - 1) / per;
    // inv = 1/(sqrt(var)+1e-6) exactly as the forward computed it
    hipLaunchKernelGGL(k_bn_inv, dim3((C + 63) / 64), dim3(64), 0, st, variance, C, w.inv);
    int rc = check_launch();
    if (rc) return rc;
    const int act = fused ? activation : ACH_LINEAR;
    hipLaunchKernelGGL(k_bn_bwd_reduce, dim3(C, nch_eff), dim3(BN_NT), 0, st, delta, x, x_norm,
                       batch, C, HW, per, mean, w.inv, scales, biases, act, w.part);
    rc = check_launch();
    if (rc) return rc;
    hipLaunchKernelGGL(k_bn_bwd_finalize, dim3((C + 63) / 64), dim3(64), 0, st, w.part, nch_eff,
                       C, batch * HW, variance, scale_updates, mean_delta, variance_delta,
                       w.coef);
    rc = check_launch();
    if (rc) return rc;
    const size_t total = (size_t)batch * C * HW;
    hipLaunchKernelGGL(k_bn_bwd_apply, dim3(grid_for(total, 256, 256u * 32u)), dim3(256), 0, st,
                       delta, x, total, C, HW, mean, w.inv, scales, biases, act, w.coef);
    return check_launch();
}

}  // extern "C"
