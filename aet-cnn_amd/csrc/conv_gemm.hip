// fp32-MFMA GEMM and implicit-GEMM convolution for gfx950.
//
// Reference behaviour replaced (paths under /root/reference/src/com/ai/dnn/):
//   Gemm.gemm                 Gemm.c:116-144     -> ach_gemm
//   conv forward GEMM loop    ConvolutionalLayer.c:716-803 -> ach_conv_fwd
//   conv weight-grad loop     ConvolutionalLayer.c:913-929 -> ach_conv_bwd_filter
//   conv input-grad + col2im  ConvolutionalLayer.c:931-945 -> ach_conv_bwd_data
// The reference runs one im2col + one GEMM per image (B launches per layer
// per pass on its GPU path).  Here each pass is ONE GEMM over the whole batch
// with the im2col gather done in the tile loader (no materialised columns):
//   forward : M = filters, N = batch*OH*OW, K = C*k*k
//   dgrad   : the forward kernel on dy with the filter flipped and
//             transposed (stride 1), pad' = k-1-pad
//   wgrad   : M = filters, N = C*k*k, K = batch*OH*OW, deterministic split-K
//             (fixed-order reduction, no float atomics)
//
// Tiling: 256 threads = 4 wave64s in a 2x2 grid; block tile 128x128x16; each
// wave owns a 64x64 sub-tile = 2x2 v_mfma_f32_32x32x2f32 accumulators (64
// VGPRs).  Global loads for tile k+1 are issued into registers before the
// MFMAs of tile k, then written to the other half of a double-buffered LDS
// stage, so one barrier per k-tile suffices.
#include "common.hpp"

namespace ach {

typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int GBM = 128, GBN = 128, GBK = 16, GNT = 256;
constexpr int LDP = 4;                 // LDS row padding (floats)
constexpr int LDA = GBM + LDP, LDB = GBN + LDP;
constexpr int RA = GBM * GBK / GNT;    // A elements per thread per k-tile (8)
constexpr int RB = GBN * GBK / GNT;    // B elements per thread per k-tile (8)

struct ConvGeom {
    int B, C, H, W;    // input
    int F, KS, S, P;   // filters, kernel, stride, pad
    int OH, OW;
};

// ---------------------------------------------------------------------------
// Thread->element maps for one k-tile.  "KC" = contiguous along k (operand
// stored with k fastest in global memory), "MC" = contiguous along m or n.
//   KC: thread t covers k = k0 + t%16 and rows r0 + t/16 + 16*i, i < 8
//   MC: thread t covers row r0 + t%128 and k = k0 + t/128 + 2*i, i < 8
__device__ __forceinline__ void lds_store_kc(float (*S)[LDA], int tid, const float *r)
{
    const int kc = tid % GBK, rr = tid / GBK;
#pragma unroll
    for (int i = 0; i < 8; ++i) S[kc][rr + 16 * i] = r[i];
}

__device__ __forceinline__ void lds_store_mc(float (*S)[LDA], int tid, const float *r)
{
    const int rc = tid % GBM, kr = tid / GBM;
#pragma unroll
    for (int i = 0; i < 8; ++i) S[kr + 2 * i][rc] = r[i];
}

// ---------------------------------------------------------------------------
// Forward implicit GEMM.  A = weights [F][C*k*k] row-major, B = im2col(x).
template <int KS_T>
struct FwdProblem {
    static constexpr bool A_KC = true, B_KC = false;
    const float *__restrict__ x;
    const float *__restrict__ w;
    float *__restrict__ y;
    ConvGeom g;
    int M, N, K;

    __device__ __forceinline__ int ks() const { return KS_T ? KS_T : g.KS; }
    __device__ __forceinline__ void krange(int, int &kb, int &ke) const { kb = 0; ke = K; }

    struct AState { int mr, kc; };
    __device__ __forceinline__ void a_init(AState &s, int m0, int tid) const
    {
        s.mr = m0 + tid / GBK;
        s.kc = tid % GBK;
    }
    __device__ __forceinline__ void a_load(const AState &s, int k0, int ke, float *r) const
    {
        const int k = k0 + s.kc;
        const bool kok = k < ke;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int m = s.mr + 16 * i;
            r[i] = (kok && m < M) ? w[(size_t)m * K + k] : 0.f;
        }
    }

    struct BState { int ok, xoff, ihb, iwb, kr; };
    __device__ __forceinline__ void b_init(BState &s, int n0, int tid) const
    {
        const int n = n0 + tid % GBN;
        s.kr = tid / GBN;
        s.ok = n < N;
        const int ohw = g.OH * g.OW;
        const int nn = s.ok ? n : 0;
        const int b = nn / ohw, p = nn - b * ohw;
        const int oh = p / g.OW, ow = p - oh * g.OW;
        s.xoff = b * g.C * g.H * g.W;
        s.ihb = oh * g.S - g.P;
        s.iwb = ow * g.S - g.P;
    }
    __device__ __forceinline__ void b_load(const BState &s, int k0, int ke, float *r) const
    {
        const int KS = ks(), KK = KS * KS;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int k = k0 + s.kr + 2 * i;
            float v = 0.f;
            if (s.ok && k < ke) {
                const int c = k / KK, t = k - c * KK;
                const int ki = t / KS, kj = t - ki * KS;
                const int ih = s.ihb + ki, iw = s.iwb + kj;
                if ((unsigned)ih < (unsigned)g.H && (unsigned)iw < (unsigned)g.W)
                    v = x[s.xoff + (c * g.H + ih) * g.W + iw];
            }
            r[i] = v;
        }
    }
    __device__ __forceinline__ void store(int m, int n, float v, int) const
    {
        if (m >= M || n >= N) return;
        const int ohw = g.OH * g.OW;
        const int b = n / ohw, p = n - b * ohw;
        y[((size_t)b * M + m) * ohw + p] = v;
    }
};

// ---------------------------------------------------------------------------
// Weight-gradient GEMM.  A = dy viewed as [F][B*OH*OW] (k = b*OHW + p),
// B[k][n] = im2col(x)[n][p] of image b, n = c*k*k + ki*k + kj.
template <int KS_T>
struct WgradProblem {
    static constexpr bool A_KC = true, B_KC = true;
    const float *__restrict__ x;
    const float *__restrict__ dy;
    float *__restrict__ dw;     // [F][C*k*k], accumulated (+=) when splits == 1
    float *__restrict__ part;   // [splits][M][N] partials when splits > 1
    ConvGeom g;
    int M, N, K, kchunk, splits;

    __device__ __forceinline__ int ks() const { return KS_T ? KS_T : g.KS; }
    __device__ __forceinline__ void krange(int z, int &kb, int &ke) const
    {
        kb = z * kchunk;
        ke = min(K, kb + kchunk);
    }

    struct AState { int mr, kc; };
    __device__ __forceinline__ void a_init(AState &s, int m0, int tid) const
    {
        s.mr = m0 + tid / GBK;
        s.kc = tid % GBK;
    }
    __device__ __forceinline__ void a_load(const AState &s, int k0, int ke, float *r) const
    {
        const int k = k0 + s.kc;
        const int ohw = g.OH * g.OW;
        const bool kok = k < ke;
        const int kk = kok ? k : 0;
        const int b = kk / ohw, p = kk - b * ohw;
        const size_t base = (size_t)b * M * ohw + p;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int m = s.mr + 16 * i;
            r[i] = (kok && m < M) ? dy[base + (size_t)m * ohw] : 0.f;
        }
    }

    struct BState { int nr, kc; };
    __device__ __forceinline__ void b_init(BState &s, int n0, int tid) const
    {
        s.nr = n0 + tid / GBK;
        s.kc = tid % GBK;
    }
    __device__ __forceinline__ void b_load(const BState &s, int k0, int ke, float *r) const
    {
        const int KS = ks(), KK = KS * KS;
        const int k = k0 + s.kc;
        const int ohw = g.OH * g.OW;
        const bool kok = k < ke;
        const int kk = kok ? k : 0;
        const int b = kk / ohw, p = kk - b * ohw;
        const int oh = p / g.OW, ow = p - oh * g.OW;
        const int ihb = oh * g.S - g.P, iwb = ow * g.S - g.P;
        const float *xb = x + (size_t)b * g.C * g.H * g.W;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int n = s.nr + 16 * i;
            float v = 0.f;
            if (kok && n < N) {
                const int c = n / KK, t = n - c * KK;
                const int ki = t / KS, kj = t - ki * KS;
                const int ih = ihb + ki, iw = iwb + kj;
                if ((unsigned)ih < (unsigned)g.H && (unsigned)iw < (unsigned)g.W)
                    v = xb[(c * g.H + ih) * g.W + iw];
            }
            r[i] = v;
        }
    }
    __device__ __forceinline__ void store(int m, int n, float v, int z) const
    {
        if (m >= M || n >= N) return;
        if (splits == 1)
            dw[(size_t)m * N + n] += v;
        else
            part[((size_t)z * M + m) * N + n] = v;
    }
};

// ---------------------------------------------------------------------------
// Plain row-major GEMM (Gemm.c:116-144): C = alpha*op(A)op(B) + beta*C.
template <bool TA, bool TB>
struct GemmProblem {
    static constexpr bool A_KC = !TA, B_KC = TB;
    const float *__restrict__ A;
    const float *__restrict__ Bm;
    float *__restrict__ C;
    int M, N, K, lda, ldb, ldc;
    float alpha, beta;

    __device__ __forceinline__ void krange(int, int &kb, int &ke) const { kb = 0; ke = K; }
    __device__ __forceinline__ float a_at(int m, int k) const
    {
        return TA ? A[(size_t)k * lda + m] : A[(size_t)m * lda + k];
    }
    __device__ __forceinline__ float b_at(int k, int n) const
    {
        return TB ? Bm[(size_t)n * ldb + k] : Bm[(size_t)k * ldb + n];
    }
    struct AState { int r, c; };
    __device__ __forceinline__ void a_init(AState &s, int m0, int tid) const
    {
        if (A_KC) { s.r = m0 + tid / GBK; s.c = tid % GBK; }
        else { s.r = m0 + tid % GBM; s.c = tid / GBM; }
    }
    __device__ __forceinline__ void a_load(const AState &s, int k0, int ke, float *r) const
    {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            int m, k;
            if (A_KC) { m = s.r + 16 * i; k = k0 + s.c; }
            else { m = s.r; k = k0 + s.c + 2 * i; }
            r[i] = (m < M && k < ke) ? a_at(m, k) : 0.f;
        }
    }
    struct BState { int r, c; };
    __device__ __forceinline__ void b_init(BState &s, int n0, int tid) const
    {
        if (B_KC) { s.r = n0 + tid / GBK; s.c = tid % GBK; }
        else { s.r = n0 + tid % GBN; s.c = tid / GBN; }
    }
    __device__ __forceinline__ void b_load(const BState &s, int k0, int ke, float *r) const
    {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            int n, k;
            if (B_KC) { n = s.r + 16 * i; k = k0 + s.c; }
            else { n = s.r; k = k0 + s.c + 2 * i; }
            r[i] = (n < N && k < ke) ? b_at(k, n) : 0.f;
        }
    }
    __device__ __forceinline__ void store(int m, int n, float v, int) const
    {
        if (m >= M || n >= N) return;
        float *cp = C + (size_t)m * ldc + n;
        *cp = (beta == 0.f) ? alpha * v : alpha * v + beta * *cp;
    }
};

// ---------------------------------------------------------------------------
template <class P>
__global__ void __launch_bounds__(GNT) k_mfma_gemm(P p)
{
    __shared__ float As[2][GBK][LDA];
    __shared__ float Bs[2][GBK][LDB];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int n0 = blockIdx.x * GBN, m0 = blockIdx.y * GBM, z = blockIdx.z;

    int kb, ke;
    p.krange(z, kb, ke);

    typename P::AState as;
    typename P::BState bs;
    p.a_init(as, m0, tid);
    p.b_init(bs, n0, tid);

    v16f acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    float ra[RA], rb[RB];
    const int nkt = (ke - kb + GBK - 1) / GBK;
    if (nkt > 0) {
        p.a_load(as, kb, ke, ra);
        p.b_load(bs, kb, ke, rb);
        if (P::A_KC) lds_store_kc(As[0], tid, ra); else lds_store_mc(As[0], tid, ra);
        if (P::B_KC) lds_store_kc(Bs[0], tid, rb); else lds_store_mc(Bs[0], tid, rb);
    }
    __syncthreads();

    const int lrow = lane >> 5, lcol = lane & 31;
    for (int kt = 0; kt < nkt; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nkt;
        if (more) {
            const int k0 = kb + (kt + 1) * GBK;
            p.a_load(as, k0, ke, ra);
            p.b_load(bs, k0, ke, rb);
        }
#pragma unroll
        for (int kk = 0; kk < GBK; kk += 2) {
            const float a0 = As[cur][kk + lrow][wm * 64 + lcol];
            const float a1 = As[cur][kk + lrow][wm * 64 + 32 + lcol];
            const float b0 = Bs[cur][kk + lrow][wn * 64 + lcol];
            const float b1 = Bs[cur][kk + lrow][wn * 64 + 32 + lcol];
            acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b0, acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b1, acc[0][1], 0, 0, 0);
            acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b0, acc[1][0], 0, 0, 0);
            acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b1, acc[1][1], 0, 0, 0);
        }
        if (more) {
            if (P::A_KC) lds_store_kc(As[cur ^ 1], tid, ra); else lds_store_mc(As[cur ^ 1], tid, ra);
            if (P::B_KC) lds_store_kc(Bs[cur ^ 1], tid, rb); else lds_store_mc(Bs[cur ^ 1], tid, rb);
        }
        __syncthreads();
    }

    // D layout of v_mfma_f32_32x32x2f32: lane l, register r holds
    // row 8*(r/4) + 4*(l/32) + r%4, column l%32.
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = n0 + wn * 64 + j * 32 + lcol;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * lrow + (r & 3);
                p.store(m, n, acc[i][j][r], z);
            }
        }
}

// Fixed-order split-K reduction: dw[i] += sum_z part[z][i], z ascending.
__global__ void k_splitk_reduce(const float *__restrict__ part, float *__restrict__ dw,
                                size_t mn, int splits)
{
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < mn;
         i += (size_t)gridDim.x * blockDim.x) {
        float s = 0.f;
        for (int z = 0; z < splits; ++z) s += part[(size_t)z * mn + i];
        dw[i] += s;
    }
}

// Wflip[c][f][a][b] = W[f][c][k-1-a][k-1-b]: turns stride-1 dgrad into a
// forward convolution of dy with C output channels.
__global__ void k_flip_weights(const float *__restrict__ w, float *__restrict__ wf,
                               int F, int C, int KS)
{
    const int KK = KS * KS;
    const size_t total = (size_t)F * C * KK;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const int t = (int)(i % KK);
        const size_t fc = i / KK;
        const int f = (int)(fc % F);
        const int c = (int)(fc / F);
        const int a = t / KS, b = t - a * KS;
        wf[i] = w[((size_t)f * C + c) * KK + (KS - 1 - a) * KS + (KS - 1 - b)];
    }
}

// ---------------------------------------------------------------------------
template <class P>
static int launch_gemm(const P &p, int M, int N, int splits, hipStream_t st)
{
    dim3 grid((N + GBN - 1) / GBN, (M + GBM - 1) / GBM, splits);
    if (grid.y > 65535u || splits > 65535) return ACH_EINVAL;
    hipLaunchKernelGGL(k_mfma_gemm<P>, grid, dim3(GNT), 0, st, p);
    return check_launch();
}

static bool conv_ok(const ach_conv_desc *d)
{
    return d && d->batch > 0 && d->c > 0 && d->h > 0 && d->w > 0 && d->n > 0 &&
           d->size > 0 && d->stride > 0 && d->pad >= 0 &&
           (d->h + 2 * d->pad - d->size) >= 0 && (d->w + 2 * d->pad - d->size) >= 0;
}

static ConvGeom geom(const ach_conv_desc *d)
{
    ConvGeom g;
    g.B = d->batch; g.C = d->c; g.H = d->h; g.W = d->w;
    g.F = d->n; g.KS = d->size; g.S = d->stride; g.P = d->pad;
    g.OH = (d->h + 2 * d->pad - d->size) / d->stride + 1;
    g.OW = (d->w + 2 * d->pad - d->size) / d->stride + 1;
    return g;
}

static bool fits_int(const ach_conv_desc *d)
{
    const ConvGeom g = geom(d);
    const double in = (double)g.B * g.C * g.H * g.W;
    const double out = (double)g.B * g.F * g.OH * g.OW;
    return in < 2147483647.0 && out < 2147483647.0 &&
           (double)g.F * g.C * g.KS * g.KS < 2147483647.0;
}

static int fwd_impl(const ConvGeom &g, const float *x, const float *w, float *y, hipStream_t st)
{
    const int M = g.F, N = g.B * g.OH * g.OW, K = g.C * g.KS * g.KS;
#define ACH_FWD(KS_)                                                        \
    {                                                                       \
        FwdProblem<KS_> p{x, w, y, g, M, N, K};                             \
        return launch_gemm(p, M, N, 1, st);                                 \
    }
    if (g.KS == 3) ACH_FWD(3)
    if (g.KS == 1) ACH_FWD(1)
    ACH_FWD(0)
#undef ACH_FWD
}

// Split count for wgrad: aim for >= ~1024 workgroups over 256 CUs, K chunks a
// multiple of the k-tile.
static void wgrad_split(const ConvGeom &g, int &splits, int &kchunk)
{
    const int M = g.F, N = g.C * g.KS * g.KS, K = g.B * g.OH * g.OW;
    const int tiles = ((M + GBM - 1) / GBM) * ((N + GBN - 1) / GBN);
    int s = (1024 + tiles - 1) / tiles;
    const int max_s = (K + 4 * GBK - 1) / (4 * GBK);  // >= 4 k-tiles per split
    if (s > max_s) s = max_s;
    if (s < 1) s = 1;
    if (s > 256) s = 256;
    int chunk = (K + s - 1) / s;
    chunk = (chunk + GBK - 1) / GBK * GBK;
    splits = (K + chunk - 1) / chunk;
    kchunk = chunk;
}

}  // namespace ach

using namespace ach;

extern "C" {

int ach_conv_out_h(const ach_conv_desc *d) { return conv_ok(d) ? geom(d).OH : -1; }
int ach_conv_out_w(const ach_conv_desc *d) { return conv_ok(d) ? geom(d).OW : -1; }

size_t ach_conv_fwd_workspace(const ach_conv_desc *) { return 0; }

int ach_conv_fwd(const ach_conv_desc *d, const float *x, const float *w, float *y,
                 void *, size_t, ach_stream_t stream)
{
    if (!conv_ok(d) || !x || !w || !y || !fits_int(d)) return ACH_EINVAL;
    return fwd_impl(geom(d), x, w, y, as_stream(stream));
}

size_t ach_conv_bwd_data_workspace(const ach_conv_desc *d)
{
    if (!conv_ok(d)) return 0;
    const ConvGeom g = geom(d);
    size_t wf = (size_t)g.F * g.C * g.KS * g.KS * sizeof(float);
    if (g.S == 1 && g.P <= g.KS - 1) return wf;
    // strided fallback: one image's column buffer
    return (size_t)g.C * g.KS * g.KS * g.OH * g.OW * sizeof(float);
}

int ach_conv_bwd_data(const ach_conv_desc *d, const float *dy, const float *w, float *dx,
                      void *ws, size_t ws_bytes, ach_stream_t stream)
{
    if (!conv_ok(d) || !dy || !w || !dx || !fits_int(d)) return ACH_EINVAL;
    const size_t need = ach_conv_bwd_data_workspace(d);
    if (!ws || ws_bytes < need) return ACH_EWORKSPACE;
    const ConvGeom g = geom(d);
    hipStream_t st = as_stream(stream);
    if (g.S == 1 && g.P <= g.KS - 1) {
        float *wf = (float *)ws;
        const size_t tot = (size_t)g.F * g.C * g.KS * g.KS;
        hipLaunchKernelGGL(k_flip_weights, dim3(grid_for(tot, 256)), dim3(256), 0, st, w, wf,
                           g.F, g.C, g.KS);
        int rc = check_launch();
        if (rc) return rc;
        ConvGeom t;
        t.B = g.B; t.C = g.F; t.H = g.OH; t.W = g.OW;
        t.F = g.C; t.KS = g.KS; t.S = 1; t.P = g.KS - 1 - g.P;
        t.OH = g.H; t.OW = g.W;
        return fwd_impl(t, dy, wf, dx, st);
    }
    // Strided convolution: the reference's per-image TN GEMM + col2im
    // (ConvolutionalLayer.c:933-945).  Not on any benchmark path.
    const int m = g.F, n = g.C * g.KS * g.KS, k = g.OH * g.OW;
    float *col = (float *)ws;
    for (int i = 0; i < g.B; ++i) {
        int rc = ach_gemm(1, 0, n, k, m, 1.f, w, n, dy + (size_t)i * m * k, k, 0.f, col, k,
                          stream);
        if (rc) return rc;
        rc = ach_col2im(col, g.C, g.H, g.W, g.KS, g.KS, g.P, g.P, g.S, g.S,
                        dx + (size_t)i * g.C * g.H * g.W, stream);
        if (rc) return rc;
    }
    return ACH_OK;
}

size_t ach_conv_bwd_filter_workspace(const ach_conv_desc *d)
{
    if (!conv_ok(d)) return 0;
    const ConvGeom g = geom(d);
    int splits, kchunk;
    wgrad_split(g, splits, kchunk);
    if (splits <= 1) return 0;
    return (size_t)splits * g.F * g.C * g.KS * g.KS * sizeof(float);
}

int ach_conv_bwd_filter(const ach_conv_desc *d, const float *x, const float *dy, float *dw,
                        void *ws, size_t ws_bytes, ach_stream_t stream)
{
    if (!conv_ok(d) || !x || !dy || !dw || !fits_int(d)) return ACH_EINVAL;
    const ConvGeom g = geom(d);
    int splits, kchunk;
    wgrad_split(g, splits, kchunk);
    const size_t need = ach_conv_bwd_filter_workspace(d);
    if (need && (!ws || ws_bytes < need)) return ACH_EWORKSPACE;
    hipStream_t st = as_stream(stream);
    const int M = g.F, N = g.C * g.KS * g.KS, K = g.B * g.OH * g.OW;
    float *part = (float *)ws;
    int rc;
#define ACH_WG(KS_)                                                         \
    {                                                                       \
        WgradProblem<KS_> p{x, dy, dw, part, g, M, N, K, kchunk, splits};   \
        rc = launch_gemm(p, M, N, splits, st);                              \
    }
    if (g.KS == 3) ACH_WG(3)
    else if (g.KS == 1) ACH_WG(1)
    else ACH_WG(0)
#undef ACH_WG
    if (rc || splits == 1) return rc;
    const size_t mn = (size_t)M * N;
    hipLaunchKernelGGL(k_splitk_reduce, dim3(grid_for(mn, 256)), dim3(256), 0, st, part, dw,
                       mn, splits);
    return check_launch();
}

int ach_gemm(int TA, int TB, int M, int N, int K, float ALPHA, const float *A, int lda,
             const float *B, int ldb, float BETA, float *C, int ldc, ach_stream_t stream)
{
    if (M < 0 || N < 0 || K < 0 || !C) return ACH_EINVAL;
    if (M == 0 || N == 0) return ACH_OK;
    if (K > 0 && (!A || !B)) return ACH_EINVAL;
    hipStream_t st = as_stream(stream);
#define ACH_GM(ta, tb)                                                              \
    {                                                                               \
        GemmProblem<ta, tb> p{A, B, C, M, N, K, lda, ldb, ldc, ALPHA, BETA};        \
        return launch_gemm(p, M, N, 1, st);                                         \
    }
    if (!TA && !TB) ACH_GM(false, false)
    if (TA && !TB) ACH_GM(true, false)
    if (!TA && TB) ACH_GM(false, true)
    ACH_GM(true, true)
#undef ACH_GM
}

}  // extern "C"
