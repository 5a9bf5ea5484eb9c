// Bandwidth-bound operators and runtime plumbing behind include/aetcnn_ops.h.
//
// Reference behaviour replaced (paths under /root/reference/src/com/ai/dnn/):
//   BLAS-1 fill/axpy/scal     mtcs/MtcsTool.c:33-132, DnnUtils.c:428-432
//   im2col / col2im           Im2Col.c:65-103, 155-192
//   add bias / bias gradient  IOData.c:43-55, BiasData.c:40-57
//   activate / gradientArray  Activation.c:160-179, 233-239
//   max-pool fwd / bwd        MaxPoolLayer.c:237-272, 318-331
//   global avg-pool fwd / bwd AvgPoolLayer.c:29-46, 73-88
//   softmax + cross-entropy   SoftMaxLayer.c:47-119
//   dropout                   DropoutLayer.c:55-86
//   SGD momentum/decay update ConvolutionalLayer.c:959-980
// All elementwise kernels are grid-stride loops over coalesced addresses;
// reductions are per-block in a fixed order (no float atomics), so every run
// is bit-reproducible.
#include "common.hpp"

#include <algorithm>
#include <float.h>
#include <stdio.h>
#include <string.h>

namespace ach {

static thread_local char g_last_err[256] = "no error";

void set_hip_error(hipError_t e)
{
    snprintf(g_last_err, sizeof(g_last_err), "%s: %s", hipGetErrorName(e),
             hipGetErrorString(e));
}

void set_error_message(const char *msg) { snprintf(g_last_err, sizeof(g_last_err), "%s", msg); }

// ---- BLAS-1 ----------------------------------------------------------------
__global__ void k_fill(float *x, size_t n, float v)
{
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        x[i] = v;
}

__global__ void k_axpy(size_t n, float a, const float *__restrict__ x, float *__restrict__ y)
{
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        y[i] += a * x[i];
}

__global__ void k_scal(size_t n, float a, float *x)
{
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        x[i] *= a;
}

// ---- im2col / col2im (one image) ----------------------------------------------
__global__ void k_im2col(const float *__restrict__ im, int C, int H, int W, int kh, int kw,
                         int ph, int pw, int sh, int sw, int dh, int dw, int OH, int OW,
                         float *__restrict__ col)
{
    const size_t total = (size_t)C * kh * kw * OH * OW;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const int ow = (int)(i % OW);
        size_t r = i / OW;
        const int oh = (int)(r % OH);
        r /= OH;
        const int kj = (int)(r % kw);
        r /= kw;
        const int ki = (int)(r % kh);
        const int c = (int)(r / kh);
        const int ih = oh * sh - ph + ki * dh, iw = ow * sw - pw + kj * dw;
        col[i] = ((unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W)
                     ? im[((size_t)c * H + ih) * W + iw]
                     : 0.f;
    }
}

// Gather form of col2im: every image pixel adds its column entries in the
// reference's (ki, kj) scan order starting from zero -> bit-identical sums
// (for one tap (ki, kj) at most one output position reads the pixel).
__global__ void k_col2im(const float *__restrict__ col, int C, int H, int W, int kh, int kw,
                         int ph, int pw, int sh, int sw, int dh, int dw, int OH, int OW,
                         float *__restrict__ im)
{
    const size_t total = (size_t)C * H * W;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const int w = (int)(i % W);
        const int h = (int)((i / W) % H);
        const int c = (int)(i / ((size_t)W * H));
        float v = 0.f;
        for (int ki = 0; ki < kh; ++ki) {
            const int t = h + ph - ki * dh;
            if (t < 0 || t % sh) continue;
            const int oh = t / sh;
            if (oh >= OH) continue;
            for (int kj = 0; kj < kw; ++kj) {
                const int u = w + pw - kj * dw;
                if (u < 0 || u % sw) continue;
                const int ow = u / sw;
                if (ow >= OW) continue;
                v += col[((((size_t)c * kh + ki) * kw + kj) * OH + oh) * OW + ow];
            }
        }
        im[i] = v;
    }
}

// ---- bias --------------------------------------------------------------------
// out[b][c][p] += bias[c]; element counts below 2^31, channel from two
// magic-number divisions
__global__ void k_add_bias(float *out, const float *__restrict__ b, int total, FastDiv dsp,
                           FastDiv dn)
{
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
        const int plane = fdiv(i, dsp);
        out[i] += b[plane - fdiv(plane, dn) * (int)dn.d];
    }
}

// Bias gradient (BiasData.calcGrad, BiasData.c:40-57): dbias[c] += sum over
// images and positions of delta.  Two passes so that every CU works: blocks
// of (channel, image chunk) write double partial sums, then one thread per
// channel adds them in chunk order (fixed order, no atomics).
constexpr int BIAS_IMGS = 8;  // images per partial-sum block

__global__ void __launch_bounds__(256) k_bias_part(const float *__restrict__ d, int batch, int n,
                                                   int spatial, double *__restrict__ part)
{
    __shared__ double sh[4];
    const int c = blockIdx.x, ch = blockIdx.y;
    const int b0 = ch * BIAS_IMGS, b1 = min(batch, b0 + BIAS_IMGS);
    double s = 0;
    const size_t plane = (size_t)n * spatial;  // image stride
    if ((spatial & 3) == 0 && (reinterpret_cast<uintptr_t>(d) & 15) == 0) {
        for (int b = b0; b < b1; ++b) {
            const float4 *p4 = reinterpret_cast<const float4 *>(d + b * plane + (size_t)c * spatial);
            for (int q = threadIdx.x; q < (spatial >> 2); q += 256) {
                const float4 v = p4[q];
                s += (double)v.x + (double)v.y + (double)v.z + (double)v.w;
            }
        }
    } else {
        // scalar planes: the chunk's images are read together so that each
        // thread has BIAS_IMGS loads in flight
        const float *p0 = d + (size_t)b0 * plane + (size_t)c * spatial;
        const int nb = b1 - b0;
        for (int q = threadIdx.x; q < spatial; q += 256) {
            float v[BIAS_IMGS];
#pragma unroll
            for (int k = 0; k < BIAS_IMGS; ++k) v[k] = k < nb ? p0[k * plane + q] : 0.f;
#pragma unroll
            for (int k = 0; k < BIAS_IMGS; ++k) s += v[k];
        }
    }
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) part[(size_t)ch * n + c] = sh[0] + sh[1] + sh[2] + sh[3];
}

// Small planes (a fully connected layer's 1x1 output): one thread per
// (channel, image chunk) sums the chunk's images x positions in order, the
// threads of a wave reading consecutive channels; k_bias_final then adds
// the chunks.
constexpr int BIAS_SMALL_SPATIAL = 16;

__global__ void __launch_bounds__(256) k_bias_small(const float *__restrict__ d, int batch, int n,
                                                    int spatial, double *__restrict__ part)
{
    const int c = blockIdx.x * blockDim.x + threadIdx.x, ch = blockIdx.y;
    if (c >= n) return;
    const int b0 = ch * BIAS_IMGS, b1 = min(batch, b0 + BIAS_IMGS);
    double s = 0;
    for (int b = b0; b < b1; ++b) {
        const float *p = d + ((size_t)b * n + c) * spatial;
        for (int q = 0; q < spatial; ++q) s += (double)p[q];
    }
    part[(size_t)ch * n + c] = s;
}

__global__ void k_bias_final(const double *__restrict__ part, int nch, int n, float *updates)
{
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= n) return;
    double s = 0;
    for (int ch = 0; ch < nch; ++ch) s += part[(size_t)ch * n + c];
    updates[c] += (float)s;
}

// ---- activations ---------------------------------------------------------------
// Streaming elementwise kernels: one float4 per thread per grid-stride step
// (float4 body when the pointers are 16-byte aligned, scalar tail), launched
// with one thread per float4 up to 2^20 blocks -- measured on MI355X as the
// fastest shape for two-input streams.
static unsigned grid_stream(size_t n) { return grid_for((n + 3) / 4, 256, 1u << 20); }

__global__ void k_activate(float *x, size_t n, int act)
{
    const size_t gid = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t done = 0;
    if ((reinterpret_cast<uintptr_t>(x) & 15) == 0) {
        float4 *x4 = reinterpret_cast<float4 *>(x);
        const size_t n4 = n >> 2;
        for (size_t i = gid; i < n4; i += stride) {
            float4 v = x4[i];
            v.x = act_forward(v.x, act); v.y = act_forward(v.y, act);
            v.z = act_forward(v.z, act); v.w = act_forward(v.w, act);
            x4[i] = v;
        }
        done = n4 << 2;
    }
    for (size_t i = done + gid; i < n; i += stride) x[i] = act_forward(x[i], act);
}

__global__ void k_gradient(const float *__restrict__ y, size_t n, int act, float *d)
{
    const size_t gid = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t done = 0;
    if (((reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(d)) & 15) == 0) {
        const float4 *y4 = reinterpret_cast<const float4 *>(y);
        float4 *d4 = reinterpret_cast<float4 *>(d);
        const size_t n4 = n >> 2;
        for (size_t i = gid; i < n4; i += stride) {
            const float4 v = y4[i];
            float4 g = d4[i];
            g.x *= act_gradient(v.x, act); g.y *= act_gradient(v.y, act);
            g.z *= act_gradient(v.z, act); g.w *= act_gradient(v.w, act);
            d4[i] = g;
        }
        done = n4 << 2;
    }
    for (size_t i = done + gid; i < n; i += stride) d[i] *= act_gradient(y[i], act);
}

// Per-plane sums of what a plane-walking kernel writes (the bias gradient's
// per-(image, channel) sums, BiasData.calcGrad BiasData.c:40-57), for a
// workgroup of 256 threads over np <= PSUM_PLANES consecutive planes walked
// flat (pixel r of the workgroup's planes at r = tid, tid + 256, ...): a
// thread's plane index never decreases, so it keeps one running double sum
// and parks it in its LDS slot red[plane][tid] when the plane changes; at
// the end one wave per plane adds the 256 slots (four per lane in order,
// then a fixed xor tree).  Deterministic.
constexpr int PSUM_PLANES = 8;
struct PlaneSum {
    double *red;  // LDS [np][256], zeroed before the walk
    int cur = -1;
    double s = 0;
    __device__ __forceinline__ void add(int pl, float v)
    {
        if (pl != cur) {
            if (cur >= 0) red[cur * 256 + threadIdx.x] = s;
            cur = pl;
            s = 0;
        }
        s += (double)v;
    }
    // every thread calls it; psum[plane0 + k] for k < np
    __device__ __forceinline__ void finish(int np, double *psum, size_t plane0)
    {
        if (cur >= 0) red[cur * 256 + threadIdx.x] = s;
        __syncthreads();
        const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
        for (int k = wave; k < np; k += 4) {
            const double *r = red + k * 256 + lane;
            double t = ((r[0] + r[64]) + r[128]) + r[192];
            t = wave_sum(t);
            if (lane == 0) psum[plane0 + k] = t;
        }
    }
};
__device__ __forceinline__ void psum_clear(double *red, int np)
{
    for (int q = threadIdx.x; q < np * 256; q += 256) red[q] = 0.0;
}

// The activation gradient (as k_gradient) of [planes][hw], one plane per
// wave, with each plane's sum of the result in psum[plane] (the bias
// gradient's per-(image, channel) sums, taken while the delta is written):
// lane l adds positions l, l + 64, ... in order (four loads in flight),
// then a fixed xor tree.  No LDS, so it fits beside the GEMMs' workgroups.
__global__ void __launch_bounds__(256) k_gradient_planes(const float *__restrict__ y, int planes,
                                                         int hw, int act, float *__restrict__ d,
                                                         double *__restrict__ psum)
{
    const int lane = threadIdx.x & 63;
    const int pl = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (pl >= planes) return;
    const size_t base = (size_t)pl * hw;
    double s = 0;
    for (int q0 = lane; q0 < hw; q0 += 4 * 64) {
        float yv[4], dv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int q = q0 + u * 64;
            yv[u] = q < hw ? y[base + q] : 0.f;
            dv[u] = q < hw ? d[base + q] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int q = q0 + u * 64;
            if (q >= hw) break;
            const float v = dv[u] * act_gradient(yv[u], act);
            d[base + q] = v;
            s += (double)v;
        }
    }
    s = wave_sum(s);
    if (lane == 0) psum[pl] = s;
}

// bias_updates[c] += sum over images b of psum[b][c] (BiasData.calcGrad's
// sums of each image's plane, BiasData.c:52-56), in double: a block takes 32
// channels, its 8 thread groups the images b = g, g + 8, ... (their loads in
// flight together), and the 8 group sums are added in group order.
constexpr int BFP_G = 8;
__global__ void __launch_bounds__(256) k_bias_from_planes(const double *__restrict__ psum,
                                                          int batch, int n, float *updates)
{
    __shared__ double sh[BFP_G][32];
    const int cl = threadIdx.x & 31, g = threadIdx.x >> 5;
    const int c = blockIdx.x * 32 + cl;
    double s = 0;
    if (c < n) {
        int b = g;
        for (; b + 3 * BFP_G < batch; b += 4 * BFP_G) {
            const double v0 = psum[(size_t)b * n + c], v1 = psum[(size_t)(b + BFP_G) * n + c];
            const double v2 = psum[(size_t)(b + 2 * BFP_G) * n + c];
            const double v3 = psum[(size_t)(b + 3 * BFP_G) * n + c];
            s = (((s + v0) + v1) + v2) + v3;
        }
        for (; b < batch; b += BFP_G) s += psum[(size_t)b * n + c];
    }
    sh[g][cl] = s;
    __syncthreads();
    if (g == 0 && c < n) {
        double t = 0;
#pragma unroll
        for (int k = 0; k < BFP_G; ++k) t += sh[k][cl];
        updates[c] += (float)t;
    }
}

// ---- max-pool --------------------------------------------------------------------
// Input element counts are below 2^31 (the indexes are int32), so all index
// arithmetic is 32-bit.
// sx_ / sy_: the width / height strides when STRIDE is 0 (else STRIDE both)
template <int SIZE, int STRIDE>
__global__ void __launch_bounds__(256) k_maxpool_fwd(const float *__restrict__ in, int total,
                                                     int H, int W, int size_, int sx_, int sy_,
                                                     int pad, FastDiv dOH, FastDiv dOW,
                                                     float *__restrict__ out,
                                                     int32_t *__restrict__ idx)
{
    const int size = SIZE ? SIZE : size_;
    const int sx = STRIDE ? STRIDE : sx_, sy = STRIDE ? STRIDE : sy_;
    const int off = -pad / 2;
    const int o = blockIdx.x * blockDim.x + threadIdx.x;
    if (o >= total) return;
    const int r = fdiv(o, dOW), j = o - r * (int)dOW.d;
    const int bc = fdiv(r, dOH), i = r - bc * (int)dOH.d;
    float mx = -FLT_MAX;
    int mi = -1;
    for (int n = 0; n < size; ++n)
        for (int m = 0; m < size; ++m) {
            const int ch = off + i * sy + n, cw = off + j * sx + m;
            const int index = cw + W * (ch + H * bc);
            const bool valid = ch >= 0 && ch < H && cw >= 0 && cw < W;
            const float v = valid ? in[index] : -FLT_MAX;
            mi = (v > mx) ? index : mi;
            mx = (v > mx) ? v : mx;
        }
    out[o] = mx;
    if (idx) idx[o] = mi;
}

// The same scan for large planes that fit in LDS: a workgroup stages ppw
// consecutive (image, channel) input planes with contiguous loads (each
// input read from HBM once, coalesced, eight loads in flight per thread),
// then every output scans its window from LDS in the same order with the
// same strict '>' -- the values and indices of k_maxpool_fwd, bit for bit,
// without its strided gathers.  Taken for output planes of at least
// POOL_FWD_MIN_OUT positions: AlexNet's 55x55 -> 27x27 pool 56 -> 42 us;
// smaller planes (27x27 -> 13x13: 28 -> 31 us, 13x13 -> 6x6: 8.8 -> 11 us
// when staged) gather faster from the caches.
constexpr int POOL_FWD_LDS_MAX = 8192;  // input floats staged per workgroup
constexpr int POOL_OUT_PER_WG = 1024;   // outputs a workgroup aims at
constexpr int POOL_FWD_MIN_OUT = 512;   // smallest output plane staged
template <int SIZE, int STRIDE>
__global__ void __launch_bounds__(256) k_maxpool_fwd_plane(const float *__restrict__ in,
                                                           int planes, int ppw, int H, int W,
                                                           int size_, int stride_, int pad,
                                                           FastDiv dOHW, FastDiv dOW,
                                                           float *__restrict__ out,
                                                           int32_t *__restrict__ idx)
{
    extern __shared__ float sp[];  // np * H * W floats
    const int size = SIZE ? SIZE : size_, stride = STRIDE ? STRIDE : stride_;
    const int off = -pad / 2, hw = H * W, ohw = (int)dOHW.d, OW = (int)dOW.d;
    const int bc0 = blockIdx.x * ppw, np = min(ppw, planes - bc0), nq = np * hw;
    const float *src = in + (size_t)bc0 * hw;
    for (int q0 = (int)threadIdx.x; q0 < nq; q0 += 8 * 256) {  // eight loads in flight
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int q = q0 + u * 256;
            v[u] = q < nq ? src[q] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int q = q0 + u * 256;
            if (q < nq) sp[q] = v[u];
        }
    }
    __syncthreads();
    for (int o = threadIdx.x; o < np * ohw; o += blockDim.x) {
        const int pl = fdiv(o, dOHW), r = o - pl * ohw;
        const int i = fdiv(r, dOW), j = r - i * OW;
        const float *pp = sp + pl * hw;
        const int gbase = (bc0 + pl) * hw;  // < 2^31: the caller's pool_ok
        float mx = -FLT_MAX;
        int mi = -1;
        for (int n = 0; n < size; ++n)
            for (int m = 0; m < size; ++m) {
                const int ch = off + i * stride + n, cw = off + j * stride + m;
                const bool valid = ch >= 0 && ch < H && cw >= 0 && cw < W;
                const float v = valid ? pp[ch * W + cw] : -FLT_MAX;
                mi = (v > mx) ? gbase + ch * W + cw : mi;
                mx = (v > mx) ? v : mx;
            }
        const size_t g = (size_t)bc0 * ohw + o;
        out[g] = mx;
        if (idx) idx[g] = mi;
    }
}

// 2x2 windows, stride 2, no offset, every window inside the image, W % 4 == 0
// (the darknet default padding = 1 on even sizes): a thread reads a 2x4 input
// block as two float4 and writes two adjacent outputs.  Same scan order and
// strict '>' as the generic kernel.
__device__ __forceinline__ void max4(float a, float b, float c, float d, int ia, int W,
                                     float &mx, int &mi)
{
    mx = -FLT_MAX;
    mi = -1;
    if (a > mx) { mx = a; mi = ia; }
    if (b > mx) { mx = b; mi = ia + 1; }
    if (c > mx) { mx = c; mi = ia + W; }
    if (d > mx) { mx = d; mi = ia + W + 1; }
}

// A dropout layer that follows a 2x2 max-pool and shares its output
// (DropoutLayer.c:55-86, NetworkFactory.c:644-650) can run inside the pool
// kernels: the forward writes r < p ? 0 : v * scale for pooled element e,
// the backward applies the same mask to the output gradient it reads
// (r = dropout_uniform(seed, iter, layer, e)) -- the values k_dropout would
// leave, bit for bit.
struct DropIn {
    float p, scale;
    uint64_t seed;
    uint32_t iter;
    uint32_t layer;
    int on;
    __device__ __forceinline__ float2 apply(float2 v, unsigned t) const
    {
        if (!on) return v;
        const uint32_t e = 2u * t;
        const float r0 = dropout_uniform(seed, iter, layer, e);
        const float r1 = dropout_uniform(seed, iter, layer, e + 1);
        v.x = (r0 < p) ? 0.f : v.x * scale;
        v.y = (r1 < p) ? 0.f : v.y * scale;
        return v;
    }
};

__global__ void __launch_bounds__(256) k_maxpool2_fwd(const float *__restrict__ in, int H, int W,
                                                      unsigned pairs, float *__restrict__ out,
                                                      int32_t *__restrict__ idx, DropIn dr)
{
    const int OW2 = W >> 2, OH = H >> 1;
    for (unsigned t = blockIdx.x * blockDim.x + threadIdx.x; t < pairs;
         t += gridDim.x * blockDim.x) {
        const int jp = (int)(t % OW2);
        const unsigned r = t / OW2;
        const int i = (int)(r % OH);
        const int bc = (int)(r / OH);
        const int i0 = (bc * H + 2 * i) * W + 4 * jp;
        const float4 a = *reinterpret_cast<const float4 *>(in + i0);
        const float4 b = *reinterpret_cast<const float4 *>(in + i0 + W);
        float2 o;
        int2 ix;
        max4(a.x, a.y, b.x, b.y, i0, W, o.x, ix.x);
        max4(a.z, a.w, b.z, b.w, i0 + 2, W, o.y, ix.y);
        reinterpret_cast<float2 *>(out)[t] = dr.apply(o, t);
        if (idx) reinterpret_cast<int2 *>(idx)[t] = ix;
    }
}

__device__ __forceinline__ int floor_div(int a, int b) { return a >= 0 ? a / b : -((-a + b - 1) / b); }

// The input gradient of a max-pool can leave the pool with the previous
// layer's activation gradient already applied (Activation.gradientArray,
// Activation.c:233-239, which that layer's backward would apply next):
// din = sum * act_gradient(y[p]), the same fp32 multiply.  y == NULL: none.
struct GradIn {
    const float *y;
    int act;
    __device__ __forceinline__ float apply(float v, size_t p) const
    {
        return y ? v * act_gradient(y[p], act) : v;
    }
};

// Gather: each input pixel visits, in ascending output order, the outputs
// whose window holds it and adds the ones whose argmax is this pixel.  With
// accumulate == 0 the sum starts from +0 instead of delta_in (the value the
// reference's zeroed delta holds), and delta_in is not read.  One thread per
// input pixel; SIZE / STRIDE are compile-time for the common windows (0 =
// taken from the arguments), which turns the window-range divisions into
// shifts.
template <int SIZE, int STRIDE>
__global__ void __launch_bounds__(256) k_maxpool_bwd(const float *__restrict__ dout,
                                                     const int32_t *__restrict__ idx, int total,
                                                     FastDiv dH, FastDiv dW, int size_,
                                                     int sx_, int sy_, int pad, int OH, int OW,
                                                     float *din, int accumulate, GradIn gi)
{
    const int size = SIZE ? SIZE : size_;
    const int sx = STRIDE ? STRIDE : sx_, sy = STRIDE ? STRIDE : sy_;
    const int p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= total) return;
    const int row = fdiv(p, dW), w = p - row * (int)dW.d;  // row = bc*H + h
    const int bc = fdiv(row, dH), h = row - bc * (int)dH.d;
    const int off = -pad / 2;
    // output row i covers rows off + i*sy .. + size-1 (columns likewise)
    const int i0 = max(floor_div(h - off - size, sy) + 1, 0);
    const int i1 = min(floor_div(h - off, sy), OH - 1);
    const int j0 = max(floor_div(w - off - size, sx) + 1, 0);
    const int j1 = min(floor_div(w - off, sx), OW - 1);
    float v = accumulate ? din[p] : 0.f;
    const int obase = bc * OH * OW;
    if constexpr (SIZE > 0 && STRIDE > 0) {
        // at most NC x NC windows hold a pixel, added in ascending output
        // order.  Every candidate's index and gradient are loaded unconditionally
        // (row / column clamped into the output plane, so each address is
        // valid) and the sum takes a hit by selection, not by branch: the
        // eight loads are in flight together.
        constexpr int NC = (SIZE + STRIDE - 1) / (STRIDE > 0 ? STRIDE : 1);
        int o[NC * NC];
        bool in[NC * NC];
        int32_t ix[NC * NC];
        float g[NC * NC];
#pragma unroll
        for (int a = 0; a < NC; ++a)
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const int i = i0 + a, j = j0 + c;
                in[a * NC + c] = i <= i1 && j <= j1;
                o[a * NC + c] = obase + min(i, OH - 1) * OW + min(j, OW - 1);
            }
#pragma unroll
        for (int q = 0; q < NC * NC; ++q) ix[q] = idx[o[q]];
#pragma unroll
        for (int q = 0; q < NC * NC; ++q) g[q] = dout[o[q]];
#pragma unroll
        for (int q = 0; q < NC * NC; ++q) {
            const float t = v + g[q];
            v = (in[q] && ix[q] == (int32_t)p) ? t : v;
        }
    } else {
        for (int i = i0; i <= i1; ++i)
            for (int j = j0; j <= j1; ++j) {
                const int o = obase + i * OW + j;
                if (idx[o] == (int32_t)p) v += dout[o];
            }
    }
    din[p] = gi.apply(v, (size_t)p);
}

// The same gather for output planes that fit in LDS: a workgroup takes ppw
// consecutive (image, channel) planes (several when planes are small, so
// that a workgroup has about a thousand input pixels), first stages their
// argmax indices and output gradients in LDS (each read from HBM once,
// coalesced), then every input pixel takes its candidates from its plane's
// LDS copy in ascending output order -- the sums of k_maxpool_bwd, bit for
// bit, without its eight dependent global loads per pixel (which stall when
// the kernel shares the CUs with a GEMM).  Dynamic LDS: 8 bytes per staged
// output position.
// With yout (the pool's forward output, unmodified since), the activation
// gradient of the layer below is taken from it: a pixel that receives a sum
// is the argmax of each window it matches, and that window's output is the
// pixel's own value, so act_gradient(yout[o]) equals act_gradient(y[p]) bit
// for bit, and a pixel that receives nothing is +0 either way (relu and
// leaky, whose gradients are finite for every input).  It reads the pooled
// tensor (a quarter of the input's size for a 3x3/2 window) instead of the
// input.  12 bytes of LDS per staged output position.
constexpr int POOL_PLANE_MAX = 4096;  // output positions staged in LDS per workgroup
constexpr int POOL_PIX_PER_WG = 1024; // input pixels a workgroup aims at
// int32 offset of k_maxpool_bwd_plane's plane-sum scratch behind its staged
// arrays of n positions (indices, gradients, and with yout the gradients of
// the activation), rounded up to 8 bytes
__host__ __device__ constexpr int pool_psum_offset(int n, bool yout)
{
    return ((yout ? 3 : 2) * n + 1) & ~1;
}

template <int SIZE, int STRIDE>
__global__ void __launch_bounds__(256) k_maxpool_bwd_plane(const float *__restrict__ dout,
                                                           const int32_t *__restrict__ idx,
                                                           FastDiv dW, FastDiv dHW, int size_,
                                                           int stride_, int pad, int OH, int OW,
                                                           int planes, int ppw, float *din,
                                                           int accumulate, GradIn gi,
                                                           double *psum, const float *yout)
{
    extern __shared__ int32_t pool_lds[];
    const int size = SIZE ? SIZE : size_, stride = STRIDE ? STRIDE : stride_;
    const int ohw = OH * OW, W = (int)dW.d, hw = (int)dHW.d;
    const int bc0 = blockIdx.x * ppw, np = min(ppw, planes - bc0);
    int32_t *six = pool_lds;
    float *sg = reinterpret_cast<float *>(pool_lds + ppw * ohw);
    // yout (optional): the pool's own output; its activation gradients are
    // staged after the gradients
    float *sgr = sg + ppw * ohw;
    // psum (optional): the sums of each input plane written, after the
    // staged arrays (rounded up to 8 bytes)
    PlaneSum ps;
    ps.red = reinterpret_cast<double *>(pool_lds + pool_psum_offset(ppw * ohw, yout != nullptr));
    if (psum) psum_clear(ps.red, np);
    const size_t obase = (size_t)bc0 * ohw;
    for (int q = threadIdx.x; q < np * ohw; q += blockDim.x) {
        six[q] = idx[obase + q];
        sg[q] = dout[obase + q];
        if (yout) sgr[q] = act_gradient(yout[obase + q], gi.act);
    }
    __syncthreads();
    const int off = -pad / 2;
    const int pbase = bc0 * hw;  // < 2^31: the caller's pool_ok
    for (int r = threadIdx.x; r < np * hw; r += blockDim.x) {
        const int pl = fdiv(r, dHW), rr = r - pl * hw;
        const int h = fdiv(rr, dW), w = rr - h * W;
        const int p = pbase + r;
        const int32_t *pix = six + pl * ohw;
        const float *pg = sg + pl * ohw;
        const float *pgr = sgr + pl * ohw;
        const int i0 = max(floor_div(h - off - size, stride) + 1, 0);
        const int i1 = min(floor_div(h - off, stride), OH - 1);
        const int j0 = max(floor_div(w - off - size, stride) + 1, 0);
        const int j1 = min(floor_div(w - off, stride), OW - 1);
        float v = accumulate ? din[p] : 0.f;
        float g = 0.f;  // with yout: the gradient at a window whose argmax is p
        if constexpr (SIZE > 0 && STRIDE > 0) {
            constexpr int NC = (SIZE + STRIDE - 1) / STRIDE;
#pragma unroll
            for (int a = 0; a < NC; ++a)
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    const int i = i0 + a, j = j0 + c;
                    if (i <= i1 && j <= j1) {
                        const int o = i * OW + j;
                        if (pix[o] == p) {
                            v += pg[o];
                            if (yout) g = pgr[o];
                        }
                    }
                }
        } else {
            for (int i = i0; i <= i1; ++i)
                for (int j = j0; j <= j1; ++j) {
                    const int o = i * OW + j;
                    if (pix[o] == p) {
                        v += pg[o];
                        if (yout) g = pgr[o];
                    }
                }
        }
        v = yout ? v * g : gi.apply(v, (size_t)p);
        din[p] = v;
        if (psum) ps.add(pl, v);
    }
    if (psum) ps.finish(np, psum, (size_t)bc0);
}

// Backward of k_maxpool2_fwd: every input pixel lies in exactly one window.
__device__ __forceinline__ float pick(float v, int p, int ix, float d)
{
    return ix == p ? v + d : v;
}

__global__ void __launch_bounds__(256) k_maxpool2_bwd(const float *__restrict__ dout,
                                                      const int32_t *__restrict__ idx, int H,
                                                      int W, unsigned pairs, float *din,
                                                      int accumulate, GradIn gi, DropIn dr)
{
    const int OW2 = W >> 2, OH = H >> 1;
    for (unsigned t = blockIdx.x * blockDim.x + threadIdx.x; t < pairs;
         t += gridDim.x * blockDim.x) {
        const int jp = (int)(t % OW2);
        const unsigned r = t / OW2;
        const int i = (int)(r % OH);
        const int bc = (int)(r / OH);
        const int i0 = (bc * H + 2 * i) * W + 4 * jp;
        const float2 d = dr.apply(reinterpret_cast<const float2 *>(dout)[t], t);
        const int2 ix = reinterpret_cast<const int2 *>(idx)[t];
        float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
        if (accumulate) {
            a = *reinterpret_cast<const float4 *>(din + i0);
            b = *reinterpret_cast<const float4 *>(din + i0 + W);
        }
        a.x = pick(a.x, i0, ix.x, d.x);         a.y = pick(a.y, i0 + 1, ix.x, d.x);
        b.x = pick(b.x, i0 + W, ix.x, d.x);     b.y = pick(b.y, i0 + W + 1, ix.x, d.x);
        a.z = pick(a.z, i0 + 2, ix.y, d.y);     a.w = pick(a.w, i0 + 3, ix.y, d.y);
        b.z = pick(b.z, i0 + W + 2, ix.y, d.y); b.w = pick(b.w, i0 + W + 3, ix.y, d.y);
        if (gi.y) {
            const float4 ya = *reinterpret_cast<const float4 *>(gi.y + i0);
            const float4 yb = *reinterpret_cast<const float4 *>(gi.y + i0 + W);
            a.x *= act_gradient(ya.x, gi.act); a.y *= act_gradient(ya.y, gi.act);
            a.z *= act_gradient(ya.z, gi.act); a.w *= act_gradient(ya.w, gi.act);
            b.x *= act_gradient(yb.x, gi.act); b.y *= act_gradient(yb.y, gi.act);
            b.z *= act_gradient(yb.z, gi.act); b.w *= act_gradient(yb.w, gi.act);
        }
        *reinterpret_cast<float4 *>(din + i0) = a;
        *reinterpret_cast<float4 *>(din + i0 + W) = b;
    }
}

// ---- global average pool -------------------------------------------------------
__global__ void k_avgpool_fwd(const float *__restrict__ in, int bc_total, int HW,
                              float *__restrict__ out)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= bc_total) return;
    const float *p = in + (size_t)i * HW;
    float s = 0.f;
    for (int k = 0; k < HW; ++k) s += p[k];
    out[i] = s / HW;
}

__global__ void k_avgpool_bwd(const float *__restrict__ dout, size_t total, int HW,
                              float *din)
{
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x)
        din[i] += dout[i / HW] / HW;
}

// ---- softmax + cross-entropy -------------------------------------------------------
// One wave per (image, group) row.  e = (float)exp(double(x/T - max/T)) as
// the reference (double exp of a float argument); p = e/sum.
__global__ void __launch_bounds__(256) k_softmax_xent(const float *__restrict__ in, int rows,
                                                      int n, float T,
                                                      const float *__restrict__ truth,
                                                      float *__restrict__ out,
                                                      float *__restrict__ delta,
                                                      float *__restrict__ err,
                                                      float *__restrict__ row_err)
{
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float *x = in + (size_t)row * n;
    float *o = out + (size_t)row * n;
    float mx = -FLT_MAX;
    for (int i = lane; i < n; i += 64) mx = fmaxf(mx, x[i]);
    mx = wave_max(mx);
    const float lt = mx / T;
    float s = 0.f;
    for (int i = lane; i < n; i += 64) {
        const float e = (float)exp((double)(x[i] / T - lt));
        o[i] = e;
        s += e;
    }
    s = wave_sum(s);
    float es = 0.f;
    for (int i = lane; i < n; i += 64) {
        const float p = o[i] / s;
        o[i] = p;
        if (truth) {
            const float t = truth[(size_t)row * n + i];
            const float e = (t != 0.f) ? -logf(p) : 0.f;
            err[(size_t)row * n + i] = e;
            delta[(size_t)row * n + i] = t - p;
            es += e;
        }
    }
    if (truth) {
        es = wave_sum(es);
        if (lane == 0) row_err[row] = es;
    }
}

// The same for rows of at least 256 classes: one 256-thread workgroup per
// row (four times the parallelism of a wave per row for the double exp),
// the four waves' max / sum / error combined through LDS in wave order.
__device__ __forceinline__ float block4_combine(float v, float *sh, bool is_max)
{
    v = is_max ? wave_max(v) : wave_sum(v);
    __syncthreads();  // sh is reused by consecutive combines
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    return is_max ? fmaxf(fmaxf(sh[0], sh[1]), fmaxf(sh[2], sh[3]))
                  : ((sh[0] + sh[1]) + sh[2]) + sh[3];
}

__global__ void __launch_bounds__(256) k_softmax_xent_row(const float *__restrict__ in, int n,
                                                          float T,
                                                          const float *__restrict__ truth,
                                                          float *__restrict__ out,
                                                          float *__restrict__ delta,
                                                          float *__restrict__ err,
                                                          float *__restrict__ row_err)
{
    __shared__ float sh[4];
    const int row = blockIdx.x;
    const float *x = in + (size_t)row * n;
    float *o = out + (size_t)row * n;
    float mx = -FLT_MAX;
    for (int i = threadIdx.x; i < n; i += 256) mx = fmaxf(mx, x[i]);
    mx = block4_combine(mx, sh, true);
    const float lt = mx / T;
    float s = 0.f;
    for (int i = threadIdx.x; i < n; i += 256) {
        const float e = (float)exp((double)(x[i] / T - lt));
        o[i] = e;
        s += e;
    }
    s = block4_combine(s, sh, false);
    float es = 0.f;
    for (int i = threadIdx.x; i < n; i += 256) {
        const float p = o[i] / s;
        o[i] = p;
        if (truth) {
            const float t = truth[(size_t)row * n + i];
            const float e = (t != 0.f) ? -logf(p) : 0.f;
            err[(size_t)row * n + i] = e;
            delta[(size_t)row * n + i] = t - p;
            es += e;
        }
    }
    if (truth) {
        es = block4_combine(es, sh, false);
        if (threadIdx.x == 0) row_err[row] = es;
    }
}

__global__ void __launch_bounds__(256) k_sum_rows(const float *__restrict__ row_err, int rows,
                                                  float *cost)
{
    __shared__ double sh[4];
    double s = 0;
    for (int i = threadIdx.x; i < rows; i += 256) s += row_err[i];
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) *cost = (float)(sh[0] + sh[1] + sh[2] + sh[3]);
}

// ---- dropout -------------------------------------------------------------------------
__device__ __forceinline__ float drop1(float v, float r, float p, float scale)
{
    return (r < p) ? 0.f : v * scale;
}

__global__ void k_dropout(float *x, size_t n, float p, float scale, uint64_t seed,
                          uint32_t iter, uint32_t layer)
{
    const size_t gid = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t done = 0;
    if ((reinterpret_cast<uintptr_t>(x) & 15) == 0) {
        float4 *x4 = reinterpret_cast<float4 *>(x);
        const size_t n4 = n >> 2;
        for (size_t i = gid; i < n4; i += stride) {
            float4 v = x4[i];
            const uint32_t e = (uint32_t)(i << 2);
            v.x = drop1(v.x, dropout_uniform(seed, iter, layer, e), p, scale);
            v.y = drop1(v.y, dropout_uniform(seed, iter, layer, e + 1), p, scale);
            v.z = drop1(v.z, dropout_uniform(seed, iter, layer, e + 2), p, scale);
            v.w = drop1(v.w, dropout_uniform(seed, iter, layer, e + 3), p, scale);
            x4[i] = v;
        }
        done = n4 << 2;
    }
    for (size_t i = done + gid; i < n; i += stride)
        x[i] = drop1(x[i], dropout_uniform(seed, iter, layer, (uint32_t)i), p, scale);
}

// ---- SGD ---------------------------------------------------------------------------------
// v += decay_coef*w; w += lr_coef*v; v *= momentum  (WeightData.c:45-78)
__device__ __forceinline__ void sgd1(float &a, float &u, float dc, float lc, float mom)
{
    sgd_step(a, u, dc, lc, mom);
}

__global__ void k_sgd(size_t n, float *__restrict__ w, float *__restrict__ v, float dc,
                      float lc, float mom)
{
    const size_t gid = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t done = 0;
    if (((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(v)) & 15) == 0) {
        float4 *w4 = reinterpret_cast<float4 *>(w);
        float4 *v4 = reinterpret_cast<float4 *>(v);
        const size_t n4 = n >> 2;
        for (size_t i = gid; i < n4; i += stride) {
            float4 a = w4[i], u = v4[i];
            sgd1(a.x, u.x, dc, lc, mom); sgd1(a.y, u.y, dc, lc, mom);
            sgd1(a.z, u.z, dc, lc, mom); sgd1(a.w, u.w, dc, lc, mom);
            w4[i] = a;
            v4[i] = u;
        }
        done = n4 << 2;
    }
    for (size_t i = done + gid; i < n; i += stride) {
        float a = w[i], u = v[i];
        sgd1(a, u, dc, lc, mom);
        w[i] = a;
        v[i] = u;
    }
}

// A layer's biases and BN scales in one launch (the two small updates of
// ConvolutionalLayer.update, ConvolutionalLayer.c:959-980, without decay):
// element i < n of (w0, v0), else element i - n of (w1, v1); the arithmetic
// of k_sgd with dc = 0.
__global__ void k_sgd_pair(int n, float *__restrict__ w0, float *__restrict__ v0,
                           float *__restrict__ w1, float *__restrict__ v1, float lc, float mom)
{
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < 2 * n; i += gridDim.x * blockDim.x) {
        const bool first = i < n;
        const int j = first ? i : i - n;
        float *w = first ? w0 : w1, *v = first ? v0 : v1;
        float a = w[j], u = v[j];
        sgd1(a, u, 0.f, lc, mom);
        w[j] = a;
        v[j] = u;
    }
}

}  // namespace ach

using namespace ach;

extern "C" {

const char *ach_version(void) { return "aetcnn-hip gfx950 0.1"; }

int ach_device_count(void)
{
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

int ach_set_device(int dev) { return check(hipSetDevice(dev)); }
const char *ach_last_hip_error(void) { return g_last_err; }

int ach_malloc(void **ptr, size_t bytes)
{
    if (!ptr) return ACH_EINVAL;
    *ptr = nullptr;
    if (bytes == 0) bytes = 256;
    return check(hipMalloc(ptr, bytes));
}

int ach_free(void *ptr) { return ptr ? check(hipFree(ptr)) : ACH_OK; }

int ach_host_alloc(void **ptr, size_t bytes)
{
    if (!ptr) return ACH_EINVAL;
    return check(hipHostMalloc(ptr, bytes ? bytes : 64, hipHostMallocDefault));
}

int ach_host_free(void *ptr) { return ptr ? check(hipHostFree(ptr)) : ACH_OK; }

int ach_memcpy_h2d(void *dst, const void *src, size_t bytes, ach_stream_t s)
{
    if (!bytes) return ACH_OK;
    if (!dst || !src) return ACH_EINVAL;
    int rc = check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(s)));
    if (rc) return rc;
    return check(hipStreamSynchronize(as_stream(s)));
}

int ach_memcpy_d2h(void *dst, const void *src, size_t bytes, ach_stream_t s)
{
    if (!bytes) return ACH_OK;
    if (!dst || !src) return ACH_EINVAL;
    int rc = check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_stream(s)));
    if (rc) return rc;
    return check(hipStreamSynchronize(as_stream(s)));
}

int ach_memcpy_h2d_async(void *dst, const void *src, size_t bytes, ach_stream_t s)
{
    if (!bytes) return ACH_OK;
    if (!dst || !src) return ACH_EINVAL;
    return check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(s)));
}

int ach_memcpy_d2d(void *dst, const void *src, size_t bytes, ach_stream_t s)
{
    if (!bytes) return ACH_OK;
    if (!dst || !src) return ACH_EINVAL;
    return check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(s)));
}

int ach_stream_create(ach_stream_t *s)
{
    if (!s) return ACH_EINVAL;
    hipStream_t st;
    int rc = check(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    *s = rc ? nullptr : (ach_stream_t)st;
    return rc;
}

int ach_stream_destroy(ach_stream_t s) { return s ? check(hipStreamDestroy(as_stream(s))) : ACH_OK; }
int ach_stream_sync(ach_stream_t s) { return check(hipStreamSynchronize(as_stream(s))); }
int ach_device_sync(void) { return check(hipDeviceSynchronize()); }

int ach_event_create(void **ev)
{
    if (!ev) return ACH_EINVAL;
    hipEvent_t e;
    int rc = check(hipEventCreate(&e));
    *ev = rc ? nullptr : (void *)e;
    return rc;
}

int ach_event_destroy(void *ev) { return ev ? check(hipEventDestroy((hipEvent_t)ev)) : ACH_OK; }

int ach_event_record(void *ev, ach_stream_t s)
{
    if (!ev) return ACH_EINVAL;
    return check(hipEventRecord((hipEvent_t)ev, as_stream(s)));
}

int ach_event_sync(void *ev)
{
    if (!ev) return ACH_EINVAL;
    return check(hipEventSynchronize((hipEvent_t)ev));
}

int ach_stream_wait_event(ach_stream_t s, void *ev)
{
    if (!ev) return ACH_EINVAL;
    return check(hipStreamWaitEvent(as_stream(s), (hipEvent_t)ev, 0));
}

int ach_event_elapsed_ms(void *a, void *b, float *ms)
{
    if (!a || !b || !ms) return ACH_EINVAL;
    int rc = check(hipEventSynchronize((hipEvent_t)b));
    if (rc) return rc;
    return check(hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b));
}

int ach_fill(float *x, size_t n, float v, ach_stream_t s)
{
    if (!n) return ACH_OK;
    if (!x) return ACH_EINVAL;
    hipLaunchKernelGGL(k_fill, dim3(grid_for(n, 256)), dim3(256), 0, as_stream(s), x, n, v);
    return check_launch();
}

int ach_axpy(size_t n, float a, const float *x, float *y, ach_stream_t s)
{
    if (!n) return ACH_OK;
    if (!x || !y) return ACH_EINVAL;
    hipLaunchKernelGGL(k_axpy, dim3(grid_for(n, 256)), dim3(256), 0, as_stream(s), n, a, x, y);
    return check_launch();
}

int ach_scal(size_t n, float a, float *x, ach_stream_t s)
{
    if (!n) return ACH_OK;
    if (!x) return ACH_EINVAL;
    hipLaunchKernelGGL(k_scal, dim3(grid_for(n, 256)), dim3(256), 0, as_stream(s), n, a, x);
    return check_launch();
}

int ach_im2col(const float *im, int C, int H, int W, int kh, int kw, int ph, int pw, int sh,
               int sw, int dh, int dw, float *col, ach_stream_t s)
{
    if (!im || !col || C <= 0 || H <= 0 || W <= 0 || kh <= 0 || kw <= 0 || sh <= 0 || sw <= 0 ||
        ph < 0 || pw < 0 || dh <= 0 || dw <= 0)
        return ACH_EINVAL;
    /* output size of the dilated window (Im2Col.c:70-73) */
    const int ekh = dh * (kh - 1) + 1, ekw = dw * (kw - 1) + 1;
    if (H + 2 * ph < ekh || W + 2 * pw < ekw) return ACH_EINVAL;
    const int OH = (H + 2 * ph - ekh) / sh + 1, OW = (W + 2 * pw - ekw) / sw + 1;
    const size_t tot = (size_t)C * kh * kw * OH * OW;
    hipLaunchKernelGGL(k_im2col, dim3(grid_for(tot, 256)), dim3(256), 0, as_stream(s), im, C, H,
                       W, kh, kw, ph, pw, sh, sw, dh, dw, OH, OW, col);
    return check_launch();
}

int ach_col2im(const float *col, int C, int H, int W, int kh, int kw, int ph, int pw, int sh,
               int sw, int dh, int dw, float *im, ach_stream_t s)
{
    if (!im || !col || C <= 0 || H <= 0 || W <= 0 || kh <= 0 || kw <= 0 || sh <= 0 || sw <= 0 ||
        ph < 0 || pw < 0 || dh <= 0 || dw <= 0)
        return ACH_EINVAL;
    const int ekh = dh * (kh - 1) + 1, ekw = dw * (kw - 1) + 1;
    if (H + 2 * ph < ekh || W + 2 * pw < ekw) return ACH_EINVAL;
    const int OH = (H + 2 * ph - ekh) / sh + 1, OW = (W + 2 * pw - ekw) / sw + 1;
    const size_t tot = (size_t)C * H * W;
    hipLaunchKernelGGL(k_col2im, dim3(grid_for(tot, 256)), dim3(256), 0, as_stream(s), col, C, H,
                       W, kh, kw, ph, pw, sh, sw, dh, dw, OH, OW, im);
    return check_launch();
}

int ach_add_bias(float *out, const float *b, int batch, int n, int spatial, ach_stream_t s)
{
    if (!out || !b || batch <= 0 || n <= 0 || spatial <= 0) return ACH_EINVAL;
    const size_t tot = (size_t)batch * n * spatial;
    if (tot >= 0x7fffffffull) return ACH_EUNSUPPORTED;
    hipLaunchKernelGGL(k_add_bias, dim3(grid_for(tot, 256, 1u << 20)), dim3(256), 0, as_stream(s),
                       out, b, (int)tot, make_fastdiv((unsigned)spatial), make_fastdiv((unsigned)n));
    return check_launch();
}

size_t ach_bias_grad_workspace(int batch, int n, int)
{
    if (batch <= 0 || n <= 0) return 0;
    const size_t nch = (size_t)(batch + BIAS_IMGS - 1) / BIAS_IMGS;
    return (nch * n * sizeof(double) + 255) & ~(size_t)255;
}

int ach_bias_grad(float *updates, const float *delta, int batch, int n, int spatial, void *ws,
                  size_t ws_bytes, ach_stream_t s)
{
    if (!updates || !delta || batch <= 0 || n <= 0 || spatial <= 0 || n > 65535) return ACH_EINVAL;
    if (!ws || ws_bytes < ach_bias_grad_workspace(batch, n, spatial)) return ACH_EWORKSPACE;
    const int nch = (batch + BIAS_IMGS - 1) / BIAS_IMGS;
    double *part = (double *)ws;
    if (spatial <= BIAS_SMALL_SPATIAL)
        hipLaunchKernelGGL(k_bias_small, dim3((n + 255) / 256, nch), dim3(256), 0, as_stream(s),
                           delta, batch, n, spatial, part);
    else
        hipLaunchKernelGGL(k_bias_part, dim3(n, nch), dim3(256), 0, as_stream(s), delta, batch, n,
                           spatial, part);
    int rc = check_launch();
    if (rc) return rc;
    hipLaunchKernelGGL(k_bias_final, dim3((n + 63) / 64), dim3(64), 0, as_stream(s), part, nch, n,
                       updates);
    return check_launch();
}

int ach_activate(float *x, size_t n, int act, ach_stream_t s)
{
    if (act == ACH_LINEAR || n == 0) return ACH_OK;  // IOData.c:68-69: LINEAR is skipped
    if (!x) return ACH_EINVAL;
    if (act != ACH_LEAKY && act != ACH_RELU && act != ACH_LOGISTIC) return ACH_EUNSUPPORTED;
    hipLaunchKernelGGL(k_activate, dim3(grid_stream(n)), dim3(256), 0, as_stream(s), x, n, act);
    return check_launch();
}

int ach_gradient(const float *y, size_t n, int act, float *d, ach_stream_t s)
{
    if (n == 0) return ACH_OK;
    if (!y || !d) return ACH_EINVAL;
    if (act == ACH_LINEAR) return ACH_OK;  // linear_gradient == 1
    if (act != ACH_LEAKY && act != ACH_RELU && act != ACH_LOGISTIC) return ACH_EUNSUPPORTED;
    hipLaunchKernelGGL(k_gradient, dim3(grid_stream(n)), dim3(256), 0, as_stream(s), y, n, act,
                       d);
    return check_launch();
}

int ach_maxpool_out(int in, int size, int stride, int padding)
{
    if (size <= 0 || stride <= 0) return -1;
    return (in + padding - size) / stride + 1;
}

static bool pool_ok(int batch, int c, int h, int w, int size, int stride, int pad)
{
    if (batch <= 0 || c <= 0 || h <= 0 || w <= 0 || size <= 0 || stride <= 0 || pad < 0)
        return false;
    if ((double)batch * c * h * w >= 2147483647.0) return false;  // int32 indexes
    return ach_maxpool_out(h, size, stride, pad) > 0 && ach_maxpool_out(w, size, stride, pad) > 0;
}

// the 2x2 / stride-2 fast path applies when the window offset is 0 and
// every window lies inside the image
static bool pool2_fast(const void *a, const void *b, int h, int w, int size, int stride, int pad,
                       int OH, int OW)
{
    return size == 2 && stride == 2 && pad / 2 == 0 && (h & 1) == 0 && (w & 3) == 0 &&
           OH == h / 2 && OW == w / 2 &&
           ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b)) & 15) == 0;
}

static int dropout_launch(float *x, size_t n, float p, uint64_t seed, uint32_t iter,
                          uint32_t layer, ach_stream_t s);

// dr.on: the following dropout runs in the 2x2 kernel, or after the pool
// on the other paths
static int maxpool_fwd(const float *in, int batch, int c, int h, int w, int size, int stride,
                       int pad, float *out, int32_t *idx, DropIn dr, ach_stream_t s)
{
    if (!in || !out || !pool_ok(batch, c, h, w, size, stride, pad)) return ACH_EINVAL;
    const int OH = ach_maxpool_out(h, size, stride, pad), OW = ach_maxpool_out(w, size, stride, pad);
    if (pool2_fast(in, out, h, w, size, stride, pad, OH, OW) &&
        (reinterpret_cast<uintptr_t>(idx) & 7) == 0) {
        const unsigned pairs = (unsigned)((size_t)batch * c * OH * OW / 2);
        hipLaunchKernelGGL(k_maxpool2_fwd, dim3(grid_for(pairs, 256, 256u * 64u)), dim3(256), 0,
                           as_stream(s), in, h, w, pairs, out, idx, dr);
        return check_launch();
    }
    if (dr.on) {
        DropIn none = dr;
        none.on = 0;
        const int rc = maxpool_fwd(in, batch, c, h, w, size, stride, pad, out, idx, none, s);
        if (rc) return rc;
        return dropout_launch(out, (size_t)batch * c * OH * OW, dr.p, dr.seed, dr.iter,
                              dr.layer, s);
    }
    const int total = batch * c * OH * OW;
    const dim3 grid((total + 255) / 256);
    const FastDiv dOH = make_fastdiv((unsigned)OH), dOW = make_fastdiv((unsigned)OW);
    if (h * w <= POOL_FWD_LDS_MAX && OH * OW >= POOL_FWD_MIN_OUT) {  // planes staged in LDS
        const int planes = batch * c;
        const int ppw = std::max(1, std::min({POOL_OUT_PER_WG / (OH * OW),
                                              POOL_FWD_LDS_MAX / (h * w), planes}));
        const dim3 pg((unsigned)((planes + ppw - 1) / ppw));
        const FastDiv dOHW = make_fastdiv((unsigned)(OH * OW));
        const size_t lds = (size_t)ppw * h * w * 4;
        if (size == 3 && stride == 2)
            hipLaunchKernelGGL((k_maxpool_fwd_plane<3, 2>), pg, dim3(256), lds, as_stream(s), in,
                               planes, ppw, h, w, size, stride, pad, dOHW, dOW, out, idx);
        else if (size == 2 && stride == 2)
            hipLaunchKernelGGL((k_maxpool_fwd_plane<2, 2>), pg, dim3(256), lds, as_stream(s), in,
                               planes, ppw, h, w, size, stride, pad, dOHW, dOW, out, idx);
        else
            hipLaunchKernelGGL((k_maxpool_fwd_plane<0, 0>), pg, dim3(256), lds, as_stream(s), in,
                               planes, ppw, h, w, size, stride, pad, dOHW, dOW, out, idx);
        return check_launch();
    }
    if (size == 3 && stride == 2)
        hipLaunchKernelGGL((k_maxpool_fwd<3, 2>), grid, dim3(256), 0, as_stream(s), in, total, h,
                           w, size, stride, stride, pad, dOH, dOW, out, idx);
    else if (size == 2 && stride == 2)
        hipLaunchKernelGGL((k_maxpool_fwd<2, 2>), grid, dim3(256), 0, as_stream(s), in, total, h,
                           w, size, stride, stride, pad, dOH, dOW, out, idx);
    else
        hipLaunchKernelGGL((k_maxpool_fwd<0, 0>), grid, dim3(256), 0, as_stream(s), in, total, h,
                           w, size, stride, stride, pad, dOH, dOW, out, idx);
    return check_launch();
}

int ach_maxpool_fwd(const float *in, int batch, int c, int h, int w, int size, int stride,
                    int pad, float *out, int32_t *idx, ach_stream_t s)
{
    DropIn none{};
    return maxpool_fwd(in, batch, c, h, w, size, stride, pad, out, idx, none, s);
}

// Unequal strides: the general window kernels (one thread per output in the
// forward, one per input pixel in the gather backward).
int ach_maxpool_fwd_xy(const float *in, int batch, int c, int h, int w, int size, int sx, int sy,
                       int pad, float *out, int32_t *idx, ach_stream_t s)
{
    if (sx == sy) return ach_maxpool_fwd(in, batch, c, h, w, size, sx, pad, out, idx, s);
    if (!in || !out || !pool_ok(batch, c, h, w, size, sx, pad) ||
        !pool_ok(batch, c, h, w, size, sy, pad))
        return ACH_EINVAL;
    const int OH = ach_maxpool_out(h, size, sy, pad), OW = ach_maxpool_out(w, size, sx, pad);
    const int total = batch * c * OH * OW;  // < 2^31: at most the input's count
    const FastDiv dOH = make_fastdiv((unsigned)OH), dOW = make_fastdiv((unsigned)OW);
    hipLaunchKernelGGL((k_maxpool_fwd<0, 0>), dim3((total + 255) / 256), dim3(256), 0,
                       as_stream(s), in, total, h, w, size, sx, sy, pad, dOH, dOW, out, idx);
    return check_launch();
}

int ach_maxpool_fwd_dropout(const float *in, int batch, int c, int h, int w, int size,
                            int stride, int pad, float *out, int32_t *idx, float probability,
                            uint64_t seed, uint32_t iter, uint32_t layer, ach_stream_t s)
{
    if (!(probability >= 0.f && probability < 1.f)) return ACH_EINVAL;
    const DropIn dr{probability, (float)(1. / (1.0 - probability)), seed, iter, layer, 1};
    return maxpool_fwd(in, batch, c, h, w, size, stride, pad, out, idx, dr, s);
}

// the planes per workgroup of k_maxpool_bwd_plane (0: output planes too
// large to stage)
static int pool_bwd_ppw(int batch, int c, int h, int w, int OH, int OW)
{
    if (OH * OW > POOL_PLANE_MAX) return 0;
    return std::max(1, std::min({POOL_PIX_PER_WG / (h * w), POOL_PLANE_MAX / (OH * OW),
                                 batch * c}));
}

// psum (optional): per-(image, channel) sums of din as written, double
// [batch][c]; only the plane-staged kernel with at most PSUM_PLANES planes
// per workgroup takes it (else ACH_EUNSUPPORTED, nothing launched).
// yout (optional): the pool's output, from which the plane-staged kernel
// takes gi's activation gradient (relu / leaky, accumulate 0; else
// ACH_EUNSUPPORTED, nothing launched)
static int maxpool_bwd(const float *dout, const int32_t *idx, int batch, int c, int h, int w,
                       int size, int stride, int pad, float *din, int accumulate, GradIn gi,
                       DropIn dr, ach_stream_t s, double *psum = nullptr,
                       const float *yout = nullptr)
{
    if (!dout || !idx || !din || !pool_ok(batch, c, h, w, size, stride, pad)) return ACH_EINVAL;
    const int OH = ach_maxpool_out(h, size, stride, pad), OW = ach_maxpool_out(w, size, stride, pad);
    const int acc = accumulate ? 1 : 0;
    if (psum || yout) {
        const int ppw = pool_bwd_ppw(batch, c, h, w, OH, OW);
        if (ppw == 0 || (psum && ppw > PSUM_PLANES) || dr.on) return ACH_EUNSUPPORTED;
        if (yout && (acc || (gi.act != ACH_RELU && gi.act != ACH_LEAKY)))
            return ACH_EUNSUPPORTED;
    }
    const bool fast2 = !psum && !yout && pool2_fast(din, dout, h, w, size, stride, pad, OH, OW) &&
                       (reinterpret_cast<uintptr_t>(idx) & 7) == 0 &&
                       (reinterpret_cast<uintptr_t>(gi.y) & 15) == 0;
    if (dr.on && !fast2) {  // the dropout backward in place on dout first
        const int rc = dropout_launch(const_cast<float *>(dout), (size_t)batch * c * OH * OW,
                                      dr.p, dr.seed, dr.iter, dr.layer, s);
        if (rc) return rc;
        dr.on = 0;
    }
    if (fast2) {
        const unsigned pairs = (unsigned)((size_t)batch * c * OH * OW / 2);
        hipLaunchKernelGGL(k_maxpool2_bwd, dim3(grid_for(pairs, 256, 256u * 64u)), dim3(256), 0,
                           as_stream(s), dout, idx, h, w, pairs, din, acc, gi, dr);
        return check_launch();
    }
    const int total = batch * c * h * w;  // < 2^31: pool_ok
    const dim3 grid((total + 255) / 256);
    const FastDiv dH = make_fastdiv((unsigned)h), dW = make_fastdiv((unsigned)w);
    if (OH * OW <= POOL_PLANE_MAX) {  // planes staged in LDS, ppw per workgroup
        const int planes = batch * c;
        const int ppw = pool_bwd_ppw(batch, c, h, w, OH, OW);
        const dim3 pg((unsigned)((planes + ppw - 1) / ppw));
        const size_t lds = (size_t)pool_psum_offset(ppw * OH * OW, yout != nullptr) * 4 +
                           (psum ? (size_t)ppw * 256 * 8 : 0);
        const FastDiv dHW = make_fastdiv((unsigned)(h * w));
        if (size == 3 && stride == 2)
            hipLaunchKernelGGL((k_maxpool_bwd_plane<3, 2>), pg, dim3(256), lds, as_stream(s), dout,
                               idx, dW, dHW, size, stride, pad, OH, OW, planes, ppw, din, acc, gi,
                               psum, yout);
        else if (size == 2 && stride == 2)
            hipLaunchKernelGGL((k_maxpool_bwd_plane<2, 2>), pg, dim3(256), lds, as_stream(s), dout,
                               idx, dW, dHW, size, stride, pad, OH, OW, planes, ppw, din, acc, gi,
                               psum, yout);
        else
            hipLaunchKernelGGL((k_maxpool_bwd_plane<0, 0>), pg, dim3(256), lds, as_stream(s), dout,
                               idx, dW, dHW, size, stride, pad, OH, OW, planes, ppw, din, acc, gi,
                               psum, yout);
        return check_launch();
    }
    if (size == 3 && stride == 2)
        hipLaunchKernelGGL((k_maxpool_bwd<3, 2>), grid, dim3(256), 0, as_stream(s), dout, idx,
                           total, dH, dW, size, stride, stride, pad, OH, OW, din, acc, gi);
    else if (size == 2 && stride == 2)
        hipLaunchKernelGGL((k_maxpool_bwd<2, 2>), grid, dim3(256), 0, as_stream(s), dout, idx,
                           total, dH, dW, size, stride, stride, pad, OH, OW, din, acc, gi);
    else
        hipLaunchKernelGGL((k_maxpool_bwd<0, 0>), grid, dim3(256), 0, as_stream(s), dout, idx,
                           total, dH, dW, size, stride, stride, pad, OH, OW, din, acc, gi);
    return check_launch();
}

int ach_maxpool_bwd(const float *dout, const int32_t *idx, int batch, int c, int h, int w,
                    int size, int stride, int pad, float *din, int accumulate, ach_stream_t s)
{
    return maxpool_bwd(dout, idx, batch, c, h, w, size, stride, pad, din, accumulate,
                       GradIn{nullptr, 0}, DropIn{}, s);
}

int ach_maxpool_bwd_xy(const float *dout, const int32_t *idx, int batch, int c, int h, int w,
                       int size, int sx, int sy, int pad, float *din, int accumulate,
                       ach_stream_t s)
{
    if (sx == sy)
        return ach_maxpool_bwd(dout, idx, batch, c, h, w, size, sx, pad, din, accumulate, s);
    if (!dout || !idx || !din || !pool_ok(batch, c, h, w, size, sx, pad) ||
        !pool_ok(batch, c, h, w, size, sy, pad))
        return ACH_EINVAL;
    const int OH = ach_maxpool_out(h, size, sy, pad), OW = ach_maxpool_out(w, size, sx, pad);
    const int total = batch * c * h * w;  // < 2^31: pool_ok
    const FastDiv dH = make_fastdiv((unsigned)h), dW = make_fastdiv((unsigned)w);
    hipLaunchKernelGGL((k_maxpool_bwd<0, 0>), dim3((total + 255) / 256), dim3(256), 0,
                       as_stream(s), dout, idx, total, dH, dW, size, sx, sy, pad, OH, OW, din,
                       accumulate ? 1 : 0, GradIn{nullptr, 0});
    return check_launch();
}

int ach_maxpool_bwd_dropout(float *dout, const int32_t *idx, int batch, int c, int h, int w,
                            int size, int stride, int pad, float *din, int accumulate,
                            float probability, uint64_t seed, uint32_t iter,
                            uint32_t layer, ach_stream_t s)
{
    if (!(probability >= 0.f && probability < 1.f)) return ACH_EINVAL;
    const DropIn dr{probability, (float)(1. / (1.0 - probability)), seed, iter, layer, 1};
    return maxpool_bwd(dout, idx, batch, c, h, w, size, stride, pad, din, accumulate,
                       GradIn{nullptr, 0}, dr, s);
}

int ach_maxpool_bwd_act(const float *dout, const int32_t *idx, int batch, int c, int h, int w,
                        int size, int stride, int pad, float *din, int accumulate,
                        const float *y_in, int act_in, ach_stream_t s)
{
    if (!y_in || (act_in != ACH_LOGISTIC && act_in != ACH_RELU && act_in != ACH_LINEAR &&
                  act_in != ACH_LEAKY))
        return ACH_EINVAL;
    return maxpool_bwd(dout, idx, batch, c, h, w, size, stride, pad, din, accumulate,
                       GradIn{y_in, act_in}, DropIn{}, s);
}

int ach_maxpool_bwd_act_planes(const float *dout, const int32_t *idx, int batch, int c, int h,
                               int w, int size, int stride, int pad, float *din,
                               const float *y_in, int act_in, double *plane_sums,
                               ach_stream_t s)
{
    if (!plane_sums || (y_in && act_in != ACH_LOGISTIC && act_in != ACH_RELU &&
                        act_in != ACH_LINEAR && act_in != ACH_LEAKY))
        return ACH_EINVAL;
    return maxpool_bwd(dout, idx, batch, c, h, w, size, stride, pad, din, 0,
                       GradIn{y_in, y_in ? act_in : ACH_LINEAR}, DropIn{}, s, plane_sums);
}

int ach_maxpool_bwd_act_pooled(const float *dout, const int32_t *idx, int batch, int c, int h,
                               int w, int size, int stride, int pad, float *din,
                               const float *pooled, int act_in, double *plane_sums,
                               ach_stream_t s)
{
    if (!pooled || (act_in != ACH_RELU && act_in != ACH_LEAKY)) return ACH_EINVAL;
    return maxpool_bwd(dout, idx, batch, c, h, w, size, stride, pad, din, 0,
                       GradIn{nullptr, act_in}, DropIn{}, s, plane_sums, pooled);
}

int ach_gradient_planes(const float *y, int batch, int n, int spatial, int act, float *delta,
                        double *plane_sums, ach_stream_t s)
{
    if (!y || !delta || !plane_sums || batch <= 0 || n <= 0 || spatial <= 0) return ACH_EINVAL;
    if (act != ACH_LEAKY && act != ACH_RELU && act != ACH_LOGISTIC && act != ACH_LINEAR)
        return ACH_EUNSUPPORTED;
    const long long planes = (long long)batch * n;
    if (planes * spatial >= 0x7fffffffll) return ACH_EUNSUPPORTED;
    hipLaunchKernelGGL(k_gradient_planes, dim3((unsigned)((planes + 3) / 4)), dim3(256), 0,
                       as_stream(s), y, (int)planes, spatial, act, delta, plane_sums);
    return check_launch();
}

int ach_bias_grad_planes(float *bias_updates, const double *plane_sums, int batch, int n,
                         ach_stream_t s)
{
    if (!bias_updates || !plane_sums || batch <= 0 || n <= 0) return ACH_EINVAL;
    hipLaunchKernelGGL(k_bias_from_planes, dim3((n + 31) / 32), dim3(256), 0, as_stream(s),
                       plane_sums, batch, n, bias_updates);
    return check_launch();
}

int ach_avgpool_fwd(const float *in, int batch, int c, int spatial, float *out, ach_stream_t s)
{
    if (!in || !out || batch <= 0 || c <= 0 || spatial <= 0) return ACH_EINVAL;
    const int bc = batch * c;
    hipLaunchKernelGGL(k_avgpool_fwd, dim3((bc + 255) / 256), dim3(256), 0, as_stream(s), in, bc,
                       spatial, out);
    return check_launch();
}

int ach_avgpool_bwd(const float *dout, int batch, int c, int spatial, float *din, ach_stream_t s)
{
    if (!dout || !din || batch <= 0 || c <= 0 || spatial <= 0) return ACH_EINVAL;
    const size_t tot = (size_t)batch * c * spatial;
    hipLaunchKernelGGL(k_avgpool_bwd, dim3(grid_for(tot, 256)), dim3(256), 0, as_stream(s), dout,
                       tot, spatial, din);
    return check_launch();
}

size_t ach_softmax_workspace(int batch, int groups)
{
    if (batch <= 0 || groups <= 0) return 0;
    return (size_t)batch * groups * sizeof(float);
}

int ach_softmax_xent(const float *in, int batch, int inputs, int groups, float T,
                     const float *truth, float *out, float *delta, float *err, float *cost,
                     void *ws, size_t ws_bytes, ach_stream_t s)
{
    if (!in || !out || batch <= 0 || inputs <= 0 || groups <= 0 || inputs % groups) return ACH_EINVAL;
    if (truth && (!delta || !err || !cost)) return ACH_EINVAL;
    const int rows = batch * groups, n = inputs / groups;
    if (truth && (!ws || ws_bytes < ach_softmax_workspace(batch, groups))) return ACH_EWORKSPACE;
    hipStream_t st = as_stream(s);
    if (n >= 256)
        hipLaunchKernelGGL(k_softmax_xent_row, dim3(rows), dim3(256), 0, st, in, n, T, truth, out,
                           delta, err, (float *)ws);
    else
        hipLaunchKernelGGL(k_softmax_xent, dim3((rows + 3) / 4), dim3(256), 0, st, in, rows, n,
                           T, truth, out, delta, err, (float *)ws);
    int rc = check_launch();
    if (rc || !truth) return rc;
    hipLaunchKernelGGL(k_sum_rows, dim3(1), dim3(256), 0, st, (const float *)ws, rows, cost);
    return check_launch();
}

float ach_dropout_uniform(uint64_t seed, uint32_t iter, uint32_t layer, uint32_t i)
{
    return dropout_uniform(seed, iter, layer, i);
}

static int dropout_launch(float *x, size_t n, float p, uint64_t seed, uint32_t iter,
                          uint32_t layer, ach_stream_t s)
{
    if (n == 0) return ACH_OK;
    if (!x || !(p >= 0.f && p < 1.f) || n > 0xffffffffull) return ACH_EINVAL;
    const float scale = (float)(1. / (1.0 - p));
    hipLaunchKernelGGL(k_dropout, dim3(grid_stream(n)), dim3(256), 0, as_stream(s), x, n, p,
                       scale, seed, iter, layer);
    return check_launch();
}

int ach_dropout_fwd(float *x, size_t n, float p, uint64_t seed, uint32_t iter, uint32_t layer,
                    ach_stream_t s)
{
    return dropout_launch(x, n, p, seed, iter, layer, s);
}

int ach_dropout_bwd(float *d, size_t n, float p, uint64_t seed, uint32_t iter, uint32_t layer,
                    ach_stream_t s)
{
    return dropout_launch(d, n, p, seed, iter, layer, s);
}

// ---- NaN scan: one workgroup per listed array ------------------------------
__global__ void __launch_bounds__(256) k_nan_scan(const ach_nan_span *__restrict__ spans,
                                                  int nspans, int32_t *flag)
{
    for (int s = blockIdx.x; s < nspans; s += gridDim.x) {
        const float *p = spans[s].p;
        const uint64_t n = spans[s].n;
        int bad = 0;
        for (uint64_t i = threadIdx.x; i < n; i += blockDim.x) bad |= isnan(p[i]);
        if (__syncthreads_or(bad) && threadIdx.x == 0) atomicMin(flag, spans[s].tag);
    }
}

int ach_nan_scan(const ach_nan_span *spans, int nspans, int32_t *flag, ach_stream_t s)
{
    if (nspans <= 0) return ACH_OK;
    if (!spans || !flag) return ACH_EINVAL;
    const int grid = nspans < 1024 ? nspans : 1024;
    hipLaunchKernelGGL(k_nan_scan, dim3(grid), dim3(256), 0, as_stream(s), spans, nspans, flag);
    return check_launch();
}

int ach_sgd_update(size_t n, float *w, float *v, float dc, float lc, float mom, ach_stream_t s)
{
    if (n == 0) return ACH_OK;
    if (!w || !v) return ACH_EINVAL;
    hipLaunchKernelGGL(k_sgd, dim3(grid_stream(n)), dim3(256), 0,
                       as_stream(s), n, w, v, dc, lc, mom);
    return check_launch();
}

int ach_conv_update(size_t nweights, float *weights, float *weight_updates, size_t n,
                    float *biases, float *bias_updates, float *scales, float *scale_updates,
                    int batch, float lr, float momentum, float decay, ach_stream_t s)
{
    if (batch <= 0) return ACH_EINVAL;
    if ((scales == nullptr) != (scale_updates == nullptr)) return ACH_EINVAL;
    const float a1 = -decay * batch;
    const float a2 = lr / batch;
    int rc = ach_sgd_update(nweights, weights, weight_updates, a1, a2, momentum, s);
    if (rc) return rc;
    if (scales && n > 0 && n <= (1u << 20)) {  // both small arrays in one launch
        if (!biases || !bias_updates) return ACH_EINVAL;
        const int n2 = (int)(2 * n);
        hipLaunchKernelGGL(k_sgd_pair, dim3((unsigned)((n2 + 255) / 256)), dim3(256), 0,
                           as_stream(s), (int)n, biases, bias_updates, scales, scale_updates, a2,
                           momentum);
        return check_launch();
    }
    rc = ach_sgd_update(n, biases, bias_updates, 0.f, a2, momentum, s);
    if (rc || !scales) return rc;
    return ach_sgd_update(n, scales, scale_updates, 0.f, a2, momentum, s);
}

}  // extern "C"
