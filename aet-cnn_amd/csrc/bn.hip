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
// Each direction is two launches:
//   reduce : grid = channels x batch chunks; each block sums its chunk of one
//            channel in double and writes one partial (no atomics);
//   apply  : grid = element chunks x channels, so the channel is uniform per
//            block; wave 0 first combines the channel's partials (the same
//            fixed-order reduction in every block, so every block derives
//            bit-identical statistics), block 0 of the channel stores the
//            per-channel results, and the block then makes one coalesced
//            elementwise pass (float4 when H*W % 4 == 0).
// Element positions are walked incrementally (no per-element division).
// The activation that follows BN in a conv layer can be fused into the
// forward apply and its gradient into both backward passes; the gradient's
// sign is taken from the recomputed BN output (same float ops as the
// forward), so the activated tensor does not have to be re-read.
#include "common.hpp"

#include <mutex>

namespace ach {

constexpr int BN_NT = 256;  // threads per block
constexpr int BN_U = 4;     // elements (float or float4) per thread in apply
// apply-pass blocks in all (each streams a contiguous share of a channel):
// the forward apply (64 VGPRs, 8 blocks per CU) in one round of 256 CUs x 8;
// the backward apply measured best at 6 per CU.  Config 2 (256 MiB tensors)
// against 4096 blocks: forward 73.7 -> 74.5%, backward 72.8 -> 75.0% of HBM;
// the darknet step unchanged within noise.
constexpr int BN_FWD_APPLY_BLOCKS = 2048;
constexpr int BN_BWD_APPLY_BLOCKS = 1536;

// reduction blocks: about BN_BWD_RED_BLOCKS (channel, image chunk) blocks
// in all for the backward reduction of tensors above BN_SMALL_ELEMS
// elements (config 2, 256 MiB tensors: 74.8% of HBM against 72.8% with 2048
// or 1024) and BN_FWD_RED_BLOCKS for smaller ones (darknet's, up to 64 MiB,
// which reduce beside the weight-gradient GEMMs: step 0.2-0.4% faster than
// with 4096, 2.2% slower with 8192); BN_FWD_RED_BLOCKS for every forward
// statistics pass (config 2: 75.1-75.5% against 73.9-74.5% with 4096; the
// darknet step unchanged).  The workspace holds the larger.
constexpr int BN_BWD_RED_BLOCKS = 4096;
constexpr int BN_FWD_RED_BLOCKS = 2048;
constexpr long long BN_SMALL_ELEMS = 1ll << 24;
static int bn_chunks(int batch, int c, int blocks = BN_BWD_RED_BLOCKS)
{
    int nch = (blocks + c - 1) / c;
    if (nch > batch) nch = batch;
    if (nch < 1) nch = 1;
    return nch;
}

template <bool VEC> struct Elem;
template <> struct Elem<true> {
    typedef float4 T;
    static constexpr int N = 4;
};
template <> struct Elem<false> {
    typedef float T;
    static constexpr int N = 1;
};

template <class T> __device__ __forceinline__ float &comp(T &v, int k)
{
    return reinterpret_cast<float *>(&v)[k];
}

// Walks positions i, i + BN_NT, ... of a channel's [batch][hwv] range:
// element (b, q) lives at ((b*C + c)*hwv + q).
struct Walk {
    int b, q, db, dq, hwv;
    __device__ __forceinline__ Walk(int i, int hwv_) : hwv(hwv_)
    {
        b = i / hwv;
        q = i - b * hwv;
        db = BN_NT / hwv;
        dq = BN_NT - db * hwv;
    }
    __device__ __forceinline__ void step()
    {
        q += dq;
        b += db;
        if (q >= hwv) {
            q -= hwv;
            ++b;
        }
    }
    __device__ __forceinline__ int at(int C, int c) const { return (b * C + c) * hwv + q; }
};

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

// Sum of partial j of channel c over the nch chunks, by one wave: lane l
// adds chunks l, l+64, ... in order, then a fixed xor tree.  Every block of
// the apply pass runs the same code on the same data, so all get the same
// bits.
__device__ __forceinline__ double chunk_sum(const double *__restrict__ part, int nch, int C, int c,
                                            int stride, int j)
{
    const int lane = threadIdx.x & 63;
    double s = 0;
    for (int ch = lane; ch < nch; ch += 64) s += part[((size_t)ch * C + c) * stride + j];
    return wave_sum(s);
}

// ---- forward statistics: partial[ch][c] = {sum x, sum x^2} -----------------
template <bool VEC>
__global__ void __launch_bounds__(BN_NT) k_bn_stats(const float *__restrict__ x, int batch,
                                                    int C, int hwv, int per,
                                                    double *__restrict__ part)
{
    typedef typename Elem<VEC>::T T;
    __shared__ double sh[BN_NT / 64];
    const int c = blockIdx.x, ch = blockIdx.y;
    const int b0 = ch * per, b1 = min(batch, b0 + per);
    const int tot = (b1 - b0) * hwv;
    const T *xv = reinterpret_cast<const T *>(x);
    double s1 = 0, s2 = 0;
    Walk wk(threadIdx.x, hwv);
    wk.b += b0;
    for (int i = threadIdx.x; i < tot; i += BN_NT * BN_U) {
        T v[BN_U];
#pragma unroll
        for (int u = 0; u < BN_U; ++u) {
            if (i + u * BN_NT < tot) v[u] = xv[wk.at(C, c)];
            wk.step();
        }
#pragma unroll
        for (int u = 0; u < BN_U; ++u) {
            if (i + u * BN_NT >= tot) continue;
#pragma unroll
            for (int k = 0; k < Elem<VEC>::N; ++k) {
                const float e = comp(v[u], k);
                s1 += (double)e;
                s2 += (double)(e * e);
            }
        }
    }
    const double t1 = block_sum<BN_NT / 64>(s1, sh);
    const double t2 = block_sum<BN_NT / 64>(s2, sh);
    if (threadIdx.x == 0) {
        part[((size_t)ch * C + c) * 2 + 0] = t1;
        part[((size_t)ch * C + c) * 2 + 1] = t2;
    }
}

// NormData.c:170-185 in float: mean = (sum x) * (1/N);
// var = (t1 + t2*mean + mean*mean*batch*spatial) * (1/(N-1)), t2 = sum(-2x)
__device__ __forceinline__ void bn_moments(double S1, double S2, int batch, int HW, float &m,
                                           float &v)
{
    const int N = batch * HW;
    const float scale = (float)(1. / N);
    m = (float)S1 * scale;
    const float t1 = (float)S2, t2 = (float)(-2.0 * S1);
    float mm = m * m;
    mm = mm * (float)batch;
    mm = mm * (float)HW;
    v = t1 + t2 * m + mm;
    v *= (float)(1. / (N - 1));
}

// NormData.c:251-262: 1/(sqrt(var) + .000001f) in double, rounded to float
__device__ __forceinline__ float bn_inv(float v)
{
    return (float)(1.0 / (sqrt((double)v) + (double)1e-6f));
}

// One block's share [per*blockIdx.x, +per) of channel c's [batch][hwv]
// range: out = act(((src - mu) * iv) * s + bb); xcopy / xnorm optional.
template <bool VEC>
__device__ __forceinline__ void bn_stream(const float *src, float *xcopy, float *xnorm,
                                          float *out, int batch, int C, int hwv, int per, int c,
                                          float mu, float iv, float s, float bb, int act)
{
    typedef typename Elem<VEC>::T T;
    const int r0 = blockIdx.x * per, r1 = min(batch * hwv, r0 + per);
    Walk wk(r0 + threadIdx.x, hwv);
    for (int i = r0 + threadIdx.x; i < r1; i += BN_NT * BN_U) {
        int at[BN_U];
        T v[BN_U];
#pragma unroll
        for (int u = 0; u < BN_U; ++u) {
            at[u] = i + u * BN_NT < r1 ? wk.at(C, c) : -1;
            wk.step();
        }
#pragma unroll
        for (int u = 0; u < BN_U; ++u)
            if (at[u] >= 0) v[u] = reinterpret_cast<const T *>(src)[at[u]];
#pragma unroll
        for (int u = 0; u < BN_U; ++u) {
            if (at[u] < 0) continue;
            if (xcopy) reinterpret_cast<T *>(xcopy)[at[u]] = v[u];
            T n, o;
#pragma unroll
            for (int k = 0; k < Elem<VEC>::N; ++k) comp(n, k) = (comp(v[u], k) - mu) * iv;
            if (xnorm) reinterpret_cast<T *>(xnorm)[at[u]] = n;
#pragma unroll
            for (int k = 0; k < Elem<VEC>::N; ++k)
                comp(o, k) = act_forward(__fmaf_rn(comp(n, k), s, bb), act);
            reinterpret_cast<T *>(out)[at[u]] = o;
        }
    }
}

// ---- forward apply ------------------------------------------------------------
// Wave 0 turns the partials into mean / variance / inv; block 0 of the
// channel writes mean, variance and the rolling statistics.  Then
// src: pre-BN tensor; xcopy (optional) gets a copy; xnorm (optional);
// out = act(xnorm*scale + bias).
template <bool VEC>
__global__ void __launch_bounds__(BN_NT) k_bn_apply(
    const float *src, float *xcopy, float *xnorm, float *out, int batch, int C, int HW, int hwv,
    int per, const double *__restrict__ part, int nch, float *__restrict__ mean,
    float *__restrict__ variance, float *__restrict__ rmean, float *__restrict__ rvar,
    const float *__restrict__ scales, const float *__restrict__ biases, int act)
{
    __shared__ float sp[2];
    const int c = blockIdx.y;
    if (threadIdx.x < 64) {
        const double S1 = chunk_sum(part, nch, C, c, 2, 0);
        const double S2 = chunk_sum(part, nch, C, c, 2, 1);
        if (threadIdx.x == 0) {
            float m, v;
            bn_moments(S1, S2, batch, HW, m, v);
            if (blockIdx.x == 0) {
                mean[c] = m;
                variance[c] = v;
                if (rmean) {
                    const float keep = .9f, take = .1f;
                    float r = rmean[c] * keep;
                    rmean[c] = r + take * m;
                    r = rvar[c] * keep;
                    rvar[c] = r + take * v;
                }
            }
            sp[0] = m;
            sp[1] = bn_inv(v);
        }
    }
    __syncthreads();
    bn_stream<VEC>(src, xcopy, xnorm, out, batch, C, hwv, per, c, sp[0], sp[1], scales[c],
                   biases[c], act);
}

// ---- forward of a small channel in one workgroup ---------------------------------
// A channel of at most BN_CH_NT*V float4 (batch*HW <= 32768 floats: darknet's
// 16x16 and 8x8 layers at batch 128) is loaded once into registers, summed
// (double: each thread's values in order, then the block's fixed tree) and
// normalized from the registers: one read and one write of the tensor in one
// launch, instead of the statistics pass, the apply pass' second read and a
// second launch.  The moments, the rolling statistics and the outputs are
// those of k_bn_stats + k_bn_apply up to the order of the double sums; src
// may be out (every thread writes only what it read, after the block's
// barrier); xcopy / xnorm optional as in k_bn_apply.
constexpr int BN_CH_NT = 1024;
constexpr int BN_CH_MAXV = 8;  // float4 per thread
template <int V>
__global__ void __launch_bounds__(BN_CH_NT) k_bn_fwd_channel(
    const float *src, float *xcopy, float *xnorm, float *out, int batch, int C, int HW, int hw4,
    float *__restrict__ mean, float *__restrict__ variance, float *__restrict__ rmean,
    float *__restrict__ rvar, const float *__restrict__ scales, const float *__restrict__ biases,
    int act)
{
    __shared__ double sh[BN_CH_NT / 64];
    __shared__ float sp[2];
    const int c = blockIdx.x, tot = batch * hw4;
    const float4 *s4 = reinterpret_cast<const float4 *>(src);
    float4 v[V];
    int at[V];
    double s1 = 0, s2 = 0;
#pragma unroll
    for (int u = 0; u < V; ++u) {
        const int e = threadIdx.x + u * BN_CH_NT, b = e / hw4;
        at[u] = e < tot ? (b * C + c) * hw4 + (e - b * hw4) : -1;
    }
#pragma unroll
    for (int u = 0; u < V; ++u)
        if (at[u] >= 0) v[u] = s4[at[u]];
#pragma unroll
    for (int u = 0; u < V; ++u) {
        if (at[u] < 0) continue;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float e = comp(v[u], k);
            s1 += (double)e;
            s2 += (double)(e * e);
        }
    }
    const double t1 = block_sum<BN_CH_NT / 64>(s1, sh);
    const double t2 = block_sum<BN_CH_NT / 64>(s2, sh);
    if (threadIdx.x == 0) {
        float m, var;
        bn_moments(t1, t2, batch, HW, m, var);
        mean[c] = m;
        variance[c] = var;
        if (rmean) {
            const float keep = .9f, take = .1f;
            float r = rmean[c] * keep;
            rmean[c] = r + take * m;
            r = rvar[c] * keep;
            rvar[c] = r + take * var;
        }
        sp[0] = m;
        sp[1] = bn_inv(var);
    }
    __syncthreads();
    const float mu = sp[0], iv = sp[1], sc = scales[c], bb = biases[c];
    float4 *o4 = reinterpret_cast<float4 *>(out);
#pragma unroll
    for (int u = 0; u < V; ++u) {
        if (at[u] < 0) continue;
        if (xcopy) reinterpret_cast<float4 *>(xcopy)[at[u]] = v[u];
        float4 n, o;
#pragma unroll
        for (int k = 0; k < 4; ++k) comp(n, k) = (comp(v[u], k) - mu) * iv;
        if (xnorm) reinterpret_cast<float4 *>(xnorm)[at[u]] = n;
#pragma unroll
        for (int k = 0; k < 4; ++k) comp(o, k) = act_forward(__fmaf_rn(comp(n, k), sc, bb), act);
        o4[at[u]] = o;
    }
}

// ---- inference ------------------------------------------------------------------
// NormData.normalizeByRoll (NormData.c:291-326): the rolling statistics
// replace the batch statistics, inv = 1/(sqrt(rolling_var) + 1e-6) in double.
template <bool VEC>
__global__ void __launch_bounds__(BN_NT) k_bn_infer(
    const float *src, float *out, int batch, int C, int hwv, int per,
    const float *__restrict__ rmean, const float *__restrict__ rvar,
    const float *__restrict__ scales, const float *__restrict__ biases, int act)
{
    const int c = blockIdx.y;
    bn_stream<VEC>(src, nullptr, nullptr, out, batch, C, hwv, per, c, rmean[c], bn_inv(rvar[c]),
                   scales[c], biases[c], act);
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
template <bool VEC>
__global__ void __launch_bounds__(BN_NT) k_bn_bwd_reduce(
    const float *__restrict__ delta, const float *__restrict__ x,
    const float *__restrict__ xnorm, int batch, int C, int hwv, int per,
    const float *__restrict__ mean, const float *__restrict__ variance,
    const float *__restrict__ scales, const float *__restrict__ biases, int act,
    double *__restrict__ part)
{
    typedef typename Elem<VEC>::T T;
    __shared__ double sh[BN_NT / 64];
    const int c = blockIdx.x, ch = blockIdx.y;
    const int b0 = ch * per, b1 = min(batch, b0 + per);
    const float mu = mean[c], iv = bn_inv(variance[c]), s = scales[c];
    const float bb = biases ? biases[c] : 0.f;
    double g1 = 0, g2 = 0, g3 = 0;
    const int tot = (b1 - b0) * hwv;
    Walk wk(threadIdx.x, hwv);
    wk.b += b0;
    constexpr int RU = BN_U / 2;  // two or three streams per element: half the batch
    for (int i = threadIdx.x; i < tot; i += BN_NT * RU) {
        T xv[RU], dv[RU], nv[RU];
#pragma unroll
        for (int u = 0; u < RU; ++u) {
            if (i + u * BN_NT < tot) {
                const int at = wk.at(C, c);
                xv[u] = reinterpret_cast<const T *>(x)[at];
                dv[u] = reinterpret_cast<const T *>(delta)[at];
                if (xnorm) nv[u] = reinterpret_cast<const T *>(xnorm)[at];
            }
            wk.step();
        }
#pragma unroll
        for (int u = 0; u < RU; ++u) {
            if (i + u * BN_NT >= tot) continue;
#pragma unroll
            for (int k = 0; k < Elem<VEC>::N; ++k) {
                const float xe = comp(xv[u], k);
                const float g = bwd_grad(comp(dv[u], k), xe, mu, iv, s, bb, act);
                const float xn = xnorm ? comp(nv[u], k) : (xe - mu) * iv;
                const float gs = g * s;
                g1 += (double)(g * xn);
                g2 += (double)gs;
                g3 += (double)(gs * (xe - mu));
            }
        }
    }
    const double t1 = block_sum<BN_NT / 64>(g1, sh);
    const double t2 = block_sum<BN_NT / 64>(g2, sh);
    const double t3 = block_sum<BN_NT / 64>(g3, sh);
    if (threadIdx.x == 0) {
        double *p = part + ((size_t)ch * C + c) * 3;
        p[0] = t1; p[1] = t2; p[2] = t3;
    }
}

// Wave 0 combines the partials into
//   scale_updates += G1; mean_delta = G2 * (-1/sqrt(var+1e-5));
//   variance_delta = G3 * (-.5 * pow(var+1e-5, -1.5))     (DeltaData.c:23-58)
// (stored by block 0 of the channel), then every element gets
//   d = d*s * 1/sqrt(v+1e-5) + vd*2*(x-mu)/N + md/N   in double (DeltaData.c:64-80).
template <bool VEC>
__global__ void __launch_bounds__(BN_NT) k_bn_bwd_apply(
    float *__restrict__ delta, const float *__restrict__ x, int batch, int C, int HW, int hwv,
    int per, const double *__restrict__ part, int nch, const float *__restrict__ mean,
    const float *__restrict__ variance, const float *__restrict__ scales,
    const float *__restrict__ biases, int act, float *__restrict__ scale_updates,
    float *__restrict__ mean_delta, float *__restrict__ variance_delta)
{
    typedef typename Elem<VEC>::T T;
    __shared__ double coef[3];
    const int c = blockIdx.y;
    if (threadIdx.x < 64) {
        const double G1 = chunk_sum(part, nch, C, c, 3, 0);
        const double G2 = chunk_sum(part, nch, C, c, 3, 1);
        const double G3 = chunk_sum(part, nch, C, c, 3, 2);
        if (threadIdx.x == 0) {
            const int N = batch * HW;
            const float ve = variance[c] + 1e-5f;
            // DeltaData.c:36  mean *= (-1./sqrt(var + 1e-5f))
            const float md = (float)((double)(float)G2 * (-1. / sqrt((double)ve)));
            // DeltaData.c:56  variance *= -.5 * pow(var + 1e-5f, -1.5f)
            const float vd =
                (float)((double)(float)G3 * (-.5 * pow((double)ve, (double)(-1.5f))));
            if (blockIdx.x == 0) {
                scale_updates[c] += (float)G1;
                if (mean_delta) mean_delta[c] = md;
                if (variance_delta) variance_delta[c] = vd;
            }
            coef[0] = 1. / sqrt((double)ve);
            coef[1] = (double)vd * 2. / (double)N;
            coef[2] = (double)(md / (float)N);
        }
    }
    __syncthreads();
    const double k0 = coef[0], k1 = coef[1], k2 = coef[2];
    const float mu = mean[c], iv = bn_inv(variance[c]), s = scales[c];
    const float bb = biases ? biases[c] : 0.f;
    const int r0 = blockIdx.x * per, r1 = min(batch * hwv, r0 + per);
    Walk wk(r0 + threadIdx.x, hwv);
    for (int i = r0 + threadIdx.x; i < r1; i += BN_NT * BN_U) {
        int at[BN_U];
        T dv[BN_U], xv[BN_U];
#pragma unroll
        for (int u = 0; u < BN_U; ++u) {
            at[u] = i + u * BN_NT < r1 ? wk.at(C, c) : -1;
            wk.step();
        }
#pragma unroll
        for (int u = 0; u < BN_U; ++u)
            if (at[u] >= 0) {
                dv[u] = reinterpret_cast<const T *>(delta)[at[u]];
                xv[u] = reinterpret_cast<const T *>(x)[at[u]];
            }
#pragma unroll
        for (int u = 0; u < BN_U; ++u) {
            if (at[u] < 0) continue;
            T o;
#pragma unroll
            for (int k = 0; k < Elem<VEC>::N; ++k) {
                const float xe = comp(xv[u], k);
                const float g = bwd_grad(comp(dv[u], k), xe, mu, iv, s, bb, act);
                const float gs = g * s;
                comp(o, k) = (float)((double)gs * k0 + k1 * (double)(xe - mu) + k2);
            }
            reinterpret_cast<T *>(delta)[at[u]] = o;
        }
    }
}

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

static size_t bn_ws_bytes(int batch, int c)
{
    return align256((size_t)bn_chunks(batch, c) * c * 3 * sizeof(double));
}

// element counts stay below 2^31 (32-bit element indexing)
static bool bn_args_ok(int batch, int c, int spatial)
{
    return batch > 0 && c > 0 && spatial > 0 && (double)batch * c * spatial < 2147483647.0 &&
           (double)batch * spatial > 1.0 && c <= 65535;
}

static bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

struct BnPlan {
    bool vec;
    int hwv, nch, per, apply_per;
    dim3 reduce_grid, apply_grid;
};

static BnPlan bn_plan(int batch, int C, int HW, bool vec_ok, int apply_blocks,
                      int red_blocks = BN_BWD_RED_BLOCKS)
{
    BnPlan p;
    p.vec = vec_ok && (HW & 3) == 0;
    p.hwv = p.vec ? HW / 4 : HW;
    const int nch = bn_chunks(batch, C, red_blocks);
    p.per = (batch + nch - 1) / nch;
    p.nch = (batch + p.per - 1) / p.per;
    p.reduce_grid = dim3(C, p.nch);
    // apply: about apply_blocks blocks in all (a block's channel statistics
    // are derived once, then it streams a contiguous share of the channel)
    const int tot = batch * p.hwv, step = BN_NT * BN_U;
    const int need = (tot + step - 1) / step;
    int chunks = (apply_blocks + C - 1) / C;
    if (chunks > need) chunks = need;
    if (chunks < 1) chunks = 1;
    p.apply_per = ((tot + chunks - 1) / chunks + step - 1) / step * step;
    p.apply_grid = dim3((tot + p.apply_per - 1) / p.apply_per, C);
    return p;
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
    double *part = (double *)ws;
    const BnPlan p = bn_plan(batch, C, HW,
                             aligned16(src) && aligned16(out) && aligned16(xcopy) &&
                                 aligned16(xnorm),
                             BN_FWD_APPLY_BLOCKS, BN_FWD_RED_BLOCKS);
    // one workgroup per channel when the channel fits its registers and the
    // channels alone give about a workgroup per CU
    const long long ch4 = (long long)batch * p.hwv;
    if (p.vec && C >= 128 && ch4 <= (long long)BN_CH_NT * BN_CH_MAXV) {
        const int V = ch4 <= BN_CH_NT ? 1 : (ch4 <= 2 * BN_CH_NT ? 2 : (ch4 <= 4 * BN_CH_NT ? 4 : 8));
        void (*kern)(const float *, float *, float *, float *, int, int, int, int, float *, float *,
                     float *, float *, const float *, const float *, int) =
            V == 1 ? k_bn_fwd_channel<1>
                   : (V == 2 ? k_bn_fwd_channel<2> : (V == 4 ? k_bn_fwd_channel<4> : k_bn_fwd_channel<8>));
        hipLaunchKernelGGL(kern, dim3(C), dim3(BN_CH_NT), 0, st, src, xcopy, xnorm, out, batch, C,
                           HW, p.hwv, mean, variance, rmean, rvar, scales, biases, act);
        return check_launch();
    }
    if (p.vec)
        hipLaunchKernelGGL(k_bn_stats<true>, p.reduce_grid, dim3(BN_NT), 0, st, src, batch, C,
                           p.hwv, p.per, part);
    else
        hipLaunchKernelGGL(k_bn_stats<false>, p.reduce_grid, dim3(BN_NT), 0, st, src, batch, C,
                           p.hwv, p.per, part);
    int rc = check_launch();
    if (rc) return rc;
    if (p.vec)
        hipLaunchKernelGGL(k_bn_apply<true>, p.apply_grid, dim3(BN_NT), 0, st, src, xcopy, xnorm,
                           out, batch, C, HW, p.hwv, p.apply_per, part, p.nch, mean, variance,
                           rmean, rvar, scales, biases, act);
    else
        hipLaunchKernelGGL(k_bn_apply<false>, p.apply_grid, dim3(BN_NT), 0, st, src, xcopy,
                           xnorm, out, batch, C, HW, p.hwv, p.apply_per, part, p.nch, mean,
                           variance, rmean, rvar, scales, biases, act);
    return check_launch();
}

/* Inference BN folded into the conv filters (ConvolutionalLayer.c:983-1003):
 * one block per filter; r = sqrt(var + 1e-5), the scale factor and the bias
 * shift in double, each result rounded once to float.  Every operation is a
 * single IEEE double op (no fused multiply-add), as in the C expression. */
__global__ void __launch_bounds__(256) k_bn_fold(int fsize, float *__restrict__ w,
                                                 float *__restrict__ b,
                                                 const float *__restrict__ scales,
                                                 const float *__restrict__ rmean,
                                                 const float *__restrict__ rvar)
{
    const int f = blockIdx.x;
    const double r = __dsqrt_rn(__dadd_rn((double)rvar[f], 1e-5));
    const double pre = __ddiv_rn((double)scales[f], r);
    float *wf = w + (size_t)f * fsize;
    for (int i = threadIdx.x; i < fsize; i += blockDim.x)
        wf[i] = (float)__dmul_rn((double)wf[i], pre);
    if (threadIdx.x == 0)
        b[f] = (float)__dsub_rn((double)b[f],
                                __ddiv_rn(__dmul_rn((double)scales[f], (double)rmean[f]), r));
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

// ---- allocation-free variant of ach_bn_train_fwd_from_x -----------------------
// The per-(channel, image chunk) partial sums live in a file-scope device
// array instead of a caller workspace.  Host code never passes the array's
// name to a kernel: its device address is looked up once per device with
// hipGetSymbolAddress (with that device current) and cached here.
static __device__ __align__(256) double scratch[ACH_BN_NOALLOC_SCRATCH_BYTES / sizeof(double)];

static double *g_scratch_dev[ACH_MAX_DEVICES];
static std::mutex g_scratch_mu;

// device address of `scratch` on the current device (nullptr on error)
static double *scratch_ptr()
{
    int dev = -1;
    if (check(hipGetDevice(&dev)) || dev < 0 || dev >= ACH_MAX_DEVICES) return nullptr;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void *p = nullptr;
        if (check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)))) return nullptr;
        g_scratch_dev[dev] = static_cast<double *>(p);
    }
    return g_scratch_dev[dev];
}

int ach_bn_train_fwd_from_x_noalloc(const float *x, float *out, int batch, int c, int spatial,
                                    const float *scales, const float *biases, float *mean,
                                    float *variance, float *rolling_mean,
                                    float *rolling_variance, int activation,
                                    ach_stream_t stream)
{
    if (!x || x == out) return ACH_EINVAL;
    if (batch <= 0 || c <= 0) return ACH_EINVAL;
    const size_t need = bn_ws_bytes(batch, c);
    if (need > ACH_BN_NOALLOC_SCRATCH_BYTES) {
        set_error_message("ach_bn_train_fwd_from_x_noalloc: the partial sums of this shape "
                          "exceed the fixed device scratch (ACH_BN_NOALLOC_SCRATCH_BYTES)");
        return ACH_EWORKSPACE;
    }
    double *ws = scratch_ptr();
    if (!ws) return ACH_EHIP;
    // every partial is written before it is read: nothing to clear
    return bn_fwd(x, nullptr, nullptr, out, batch, c, spatial, scales, biases, mean, variance,
                  rolling_mean, rolling_variance, activation, ws, need, as_stream(stream));
}

int ach_bn_infer(const float *x, float *out, int batch, int c, int spatial,
                 const float *scales, const float *biases, const float *rolling_mean,
                 const float *rolling_variance, int activation, ach_stream_t stream)
{
    if (!bn_args_ok(batch, c, spatial) || !x || !out || !scales || !biases || !rolling_mean ||
        !rolling_variance)
        return ACH_EINVAL;
    const BnPlan p = bn_plan(batch, c, spatial, aligned16(x) && aligned16(out), BN_FWD_APPLY_BLOCKS);
    hipStream_t st = as_stream(stream);
    if (p.vec)
        hipLaunchKernelGGL(k_bn_infer<true>, p.apply_grid, dim3(BN_NT), 0, st, x, out, batch, c,
                           p.hwv, p.apply_per, rolling_mean, rolling_variance, scales, biases,
                           activation);
    else
        hipLaunchKernelGGL(k_bn_infer<false>, p.apply_grid, dim3(BN_NT), 0, st, x, out, batch, c,
                           p.hwv, p.apply_per, rolling_mean, rolling_variance, scales, biases,
                           activation);
    return check_launch();
}

int ach_conv_bn_fold(int filters, int fsize, float *weights, float *biases,
                     const float *scales, const float *rolling_mean,
                     const float *rolling_variance, ach_stream_t stream)
{
    if (filters <= 0 || fsize <= 0 || filters > 65535 || !weights || !biases || !scales ||
        !rolling_mean || !rolling_variance)
        return ACH_EINVAL;
    hipLaunchKernelGGL(k_bn_fold, dim3(filters), dim3(256), 0, as_stream(stream), fsize,
                       weights, biases, scales, rolling_mean, rolling_variance);
    return check_launch();
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
    double *part = (double *)ws;
    const bool small = (long long)batch * C * HW <= BN_SMALL_ELEMS;
    const BnPlan p = bn_plan(batch, C, HW, aligned16(delta) && aligned16(x) && aligned16(x_norm),
                             BN_BWD_APPLY_BLOCKS, small ? BN_FWD_RED_BLOCKS : BN_BWD_RED_BLOCKS);
    const int act = fused ? activation : ACH_LINEAR;
    if (p.vec)
        hipLaunchKernelGGL(k_bn_bwd_reduce<true>, p.reduce_grid, dim3(BN_NT), 0, st, delta, x,
                           x_norm, batch, C, p.hwv, p.per, mean, variance, scales, biases, act,
                           part);
    else
        hipLaunchKernelGGL(k_bn_bwd_reduce<false>, p.reduce_grid, dim3(BN_NT), 0, st, delta, x,
                           x_norm, batch, C, p.hwv, p.per, mean, variance, scales, biases, act,
                           part);
    int rc = check_launch();
    if (rc) return rc;
    if (p.vec)
        hipLaunchKernelGGL(k_bn_bwd_apply<true>, p.apply_grid, dim3(BN_NT), 0, st, delta, x,
                           batch, C, HW, p.hwv, p.apply_per, part, p.nch, mean, variance, scales,
                           biases, act, scale_updates, mean_delta, variance_delta);
    else
        hipLaunchKernelGGL(k_bn_bwd_apply<false>, p.apply_grid, dim3(BN_NT), 0, st, delta, x,
                           batch, C, HW, p.hwv, p.apply_per, part, p.nch, mean, variance, scales,
                           biases, act, scale_updates, mean_delta, variance_delta);
    return check_launch();
}

}  // extern "C"
