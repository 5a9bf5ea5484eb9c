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
// Kernel shape: 256 threads = 4 wave64s; block tile BM x 128 x BK; each wave
// owns a (BM/WM) x (128/WN) sub-tile of v_mfma_f32_32x32x2f32 accumulators.
// Operands are fetched with buffer loads whose out-of-range offsets return
// zero in hardware, so padding, ragged K and partial tiles cost no branches.
// The global loads of k-tile t+1 are issued among the MFMAs of the first two
// k-steps of tile t and written to the other half of a double-buffered LDS
// stage among the MFMAs of its last k-step (one barrier per k-tile); the
// scheduler is told to interleave them with the MFMAs so they issue in the
// matrix pipe's shadow.  For 3x3 filters the k-tile is 18 = two input
// channels, which makes the im2col (ki, kj) of every loaded row a
// compile-time constant.  Workgroups are remapped so that neighbouring
// tiles of one K slice (M-tiles sharing an input patch, N-tiles sharing a
// delta slice) run on the same XCD and share its L2.
#include "common.hpp"

#include <type_traits>

namespace ach {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));

constexpr int GNT = 256;     // threads per workgroup
// thread index within a GNT-thread group: a GEMM workgroup may hold
// several groups, each loading its own operand tiles
__device__ __forceinline__ int ltid() { return (int)(threadIdx.x & (GNT - 1)); }
constexpr int GBN = 128;     // N tile
constexpr int LDP = 4;       // LDS row padding (floats)
// The forward loaders' operand rows (AWeightsT, AWeightsT4, BIm2col3,
// BIm2colK, BIm2colAny) are unpadded: 128 floats, so every k-step's fragment
// pair sits a whole number of 64-float units from one base and one
// ds_read2st64 reads it without address arithmetic.  Their stores write whole
// 64-lane row segments (no conflicts).
constexpr int LDP_FWD = 0;
constexpr unsigned kOOB = 0x80000000u;  // buffer offset that reads as 0
constexpr int WGRAD_BK = 16;            // k-tile of the weight-gradient GEMM
// weight-gradient workgroups aimed for (tiles x splits) in the (image,
// position) K order
constexpr int WGRAD_TARGET = 2048;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, unsigned bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes,
                                             0x00020000);
}

// element offset -> byte offset, or the out-of-range offset when invalid
__device__ __forceinline__ int boff(bool ok, int elem)
{
    return ok ? elem * 4 : (int)kOOB;
}

// the builtin returns the loaded dword as an integer: reinterpret its bits
__device__ __forceinline__ float bload(__amdgpu_buffer_rsrc_t r, int byte_off)
{
    return __int_as_float((int)__builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, 0));
}

// The same with a wave-uniform byte offset in the instruction's scalar
// offset operand (an SGPR): loaders with loop-invariant per-thread offsets
// add the k-tile's uniform advance there instead of in one VGPR per load.
// Callers keep voff + soff inside the buffer for every in-range voff (the
// prefetch past the last k-tile re-reads the last tile), so the address is
// valid whether or not the range check includes the scalar offset; an
// out-of-range voff (>= 2^31) reads zero either way.
__device__ __forceinline__ float bload_so(__amdgpu_buffer_rsrc_t r, unsigned voff, unsigned soff)
{
    return __int_as_float(
        (int)__builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0));
}


struct ConvGeom {
    int B, C, H, W;    // input
    int F, KS, S, P;   // filters, kernel, stride, pad
    int OH, OW;
    FastDiv dkk, dks;  // division by KS*KS and by KS
};

// ===========================================================================
// Operand loaders.  Each provides, for its k-tile width BK:
//   RA / RB          elements per thread per k-tile
//   init(m0|n0,tid)  loop-invariant per-thread state
//   load(k0, ke, r)  global -> registers for k in [k0, k0+BK) clipped to ke
//   store(S, r)      registers -> LDS stage S[BK][BM or BN + LDP]
// ===========================================================================

// A = weights stored k-major, Wt[K][M] (m contiguous): thread -> column
// m0 + tid%BM, rows tid/BM + (256/BM)*i.  Loads are coalesced along m and
// the LDS stores hit consecutive banks.
template <int BM, int BK>
struct AWeightsT {
    static constexpr int RPI = GNT / BM;                 // rows per step
    static constexpr int RA = (BK + RPI - 1) / RPI, PAD = LDP_FWD;
    __amdgpu_buffer_rsrc_t rs;
    int M, mok, kr, col;
    __device__ __forceinline__ void init(const float *wt, int M_, int K_, int m0, int tid)
    {
        M = M_;
        rs = make_rsrc(wt, (unsigned)((size_t)M_ * K_ * 4));
        col = m0 + tid % BM;
        kr = tid / BM;
        mok = col < M_;
    }
    __device__ __forceinline__ void load(int k0, int ke, float *ra) const
    {
#pragma unroll
        for (int i = 0; i < RA; ++i) {
            const int k = k0 + kr + RPI * i;
            ra[i] = bload(rs, boff(mok && k < ke && kr + RPI * i < BK, k * M + col));
        }
    }
    template <int LD>
    __device__ __forceinline__ void store(float (*S)[LD], const float *ra) const
    {
        const int mc = ltid() % BM;
#pragma unroll
        for (int i = 0; i < RA; ++i)
            if (kr + RPI * i < BK) S[kr + RPI * i][mc] = ra[i];
    }
};

// The same k-major weights read as float4 when M % 4 == 0: thread -> float4
// f = tid + 256*i of the BK x BM tile (row f / (BM/4), columns 4*(f % (BM/4))
// .. +3), one dwordx4 buffer load and one 16-byte LDS store each, instead of
// four dword loads and stores.
__device__ __forceinline__ float4 bload4(__amdgpu_buffer_rsrc_t r, int byte_off)
{
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0);
    return make_float4(__int_as_float((int)v[0]), __int_as_float((int)v[1]),
                       __int_as_float((int)v[2]), __int_as_float((int)v[3]));
}

__device__ __forceinline__ float4 bload4_so(__amdgpu_buffer_rsrc_t r, unsigned voff, unsigned soff)
{
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
    return make_float4(__int_as_float((int)v[0]), __int_as_float((int)v[1]),
                       __int_as_float((int)v[2]), __int_as_float((int)v[3]));
}

template <int BM, int BK>
struct AWeightsT4 {
    static constexpr bool SPILL = BK == 18;
    static constexpr int C4 = BM / 4;                      // float4 per tile row
    static constexpr int NV = (BK * C4 + GNT - 1) / GNT;   // float4 per thread
    static constexpr int RA = 4 * NV, PAD = LDP_FWD;
    static_assert(BM % 4 == 0 && ((BM + PAD) % 4) == 0, "16-byte LDS rows");
    __amdgpu_buffer_rsrc_t rs;
    int M, m0;
    __device__ __forceinline__ void init(const float *wt, int M_, int K_, int m0_, int)
    {
        M = M_;
        m0 = m0_;
        rs = make_rsrc(wt, (unsigned)((size_t)M_ * K_ * 4));
    }
    __device__ __forceinline__ void load(int k0, int ke, float *ra) const
    {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int f = ltid() + GNT * i;
            const int row = f / C4, m = m0 + 4 * (f % C4), k = k0 + row;
            const bool ok = f < BK * C4 && k < ke && m < M;
            const float4 v = bload4(rs, boff(ok, k * M + m));
            ra[4 * i] = v.x; ra[4 * i + 1] = v.y; ra[4 * i + 2] = v.z; ra[4 * i + 3] = v.w;
        }
    }
    // The last pass may run past the BK rows of the stage (BK*C4 not a
    // multiple of 256: 18 x 32 float4 for 3x3 filters and 128-row tiles).
    // With SPILL (the 3x3 k-tiles) those lanes store to a 1 KB slot that
    // nobody reads (shared by the overflowing waves) instead of branching
    // around the store, so the store stays in the MFMA interleave and the
    // barrier no longer waits for it: darknet step -0.4%, AlexNet unchanged;
    // the 5x5 k-tiles (BK = 26) keep the branch (AlexNet +0.3% with it).
    // (Allocating the overflow rows instead cost 6 of the 24 A rows of LDS
    // and left 3 128-row workgroups per CU instead of 4.)
    template <int LD>
    __device__ __forceinline__ void store(float (*S)[LD], const float *ra) const
    {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int f = ltid() + GNT * i;
            const float4 v = make_float4(ra[4 * i], ra[4 * i + 1], ra[4 * i + 2], ra[4 * i + 3]);
            if (i + 1 < NV || NV * GNT <= BK * C4) {
                *reinterpret_cast<float4 *>(&S[f / C4][4 * (f % C4)]) = v;
            } else if constexpr (!SPILL) {
                if (f < BK * C4) *reinterpret_cast<float4 *>(&S[f / C4][4 * (f % C4)]) = v;
            } else {
                __shared__ float4 spill[64];
                float4 *dst = f < BK * C4 ? reinterpret_cast<float4 *>(&S[f / C4][4 * (f % C4)])
                                          : &spill[threadIdx.x & 63];
                *dst = v;
            }
        }
    }
};

// A = a filter in its own layout W[M][K] (k contiguous: the fully
// connected layers, whose k-major copy would cost a pass over the largest
// weights every step).  Thread -> float4 f = tid + 256*i of the BM x BK tile
// (row m0 + f / (BK/4), k 4*(f % (BK/4)) .. +3): one dwordx4 load when K % 4
// == 0 (16-byte aligned rows), four dword loads otherwise; the four values
// go to four LDS rows of the k-major stage.
template <int BM, int BK>
struct AWeightsN {
    static constexpr int K4 = BK / 4;                      // float4 per tile row
    static constexpr int NV = (BM * K4 + GNT - 1) / GNT;   // float4 per thread
    static constexpr int RA = 4 * NV, PAD = LDP;
    static_assert(BK % 4 == 0, "k-tile of whole float4");
    __amdgpu_buffer_rsrc_t rs;
    int M, K, m0;
    bool v4;
    __device__ __forceinline__ void init(const float *w, int M_, int K_, int m0_, int)
    {
        M = M_;
        K = K_;
        m0 = m0_;
        v4 = (K_ & 3) == 0;
        rs = make_rsrc(w, (unsigned)((size_t)M_ * K_ * 4));
    }
    __device__ __forceinline__ void load(int k0, int ke, float *ra) const
    {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int f = ltid() + GNT * i;
            const int m = m0 + f / K4, k = k0 + 4 * (f % K4);
            const bool ok = f < BM * K4 && m < M;
            if (v4) {
                const float4 v = bload4(rs, boff(ok && k < ke, m * K + k));
                ra[4 * i] = v.x; ra[4 * i + 1] = v.y; ra[4 * i + 2] = v.z; ra[4 * i + 3] = v.w;
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    ra[4 * i + j] = bload(rs, boff(ok && k + j < ke, m * K + k + j));
            }
        }
    }
    template <int LD>
    __device__ __forceinline__ void store(float (*S)[LD], const float *ra) const
    {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int f = ltid() + GNT * i;
            if (f < BM * K4) {
                const int mc = f / K4, kc = 4 * (f % K4);
#pragma unroll
                for (int j = 0; j < 4; ++j) S[kc + j][mc] = ra[4 * i + j];
            }
        }
    }
};

// AWeightsT4 for problems whose every k-tile is full (K a multiple of BK):
// the per-thread byte offsets of the NV float4 (or the out-of-range offset
// for columns past M and rows past BK) are loop-invariant, and a k-tile only
// adds the uniform k0*M*4 (the scalar offset).  The prefetch after the last
// tile (k0 >= ke) re-reads the last tile; those values are never used.
template <int BM, int BK>
struct AWeightsT4F : AWeightsT4<BM, BK> {
    using Base = AWeightsT4<BM, BK>;
    using Base::NV;
    using Base::C4;
    unsigned voff[NV];
    int M4;
    __device__ __forceinline__ void init(const float *wt, int M_, int K_, int m0_, int)
    {
        Base::init(wt, M_, K_, m0_, 0);
        M4 = M_ * 4;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int f = ltid() + GNT * i;
            const int row = f / C4, m = m0_ + 4 * (f % C4);
            voff[i] = (f < BK * C4 && m < M_) ? (unsigned)(row * M_ + m) * 4u : kOOB;
        }
    }
    __device__ __forceinline__ void load(int k0, int ke, float *ra) const
    {
        const unsigned d = (unsigned)((k0 < ke ? k0 : k0 - BK) * M4);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const float4 v = bload4_so(this->rs, voff[i], d);
            ra[4 * i] = v.x; ra[4 * i + 1] = v.y; ra[4 * i + 2] = v.z; ra[4 * i + 3] = v.w;
        }
    }
};

// B for the forward pass with a 3x3 kernel and BK = 9*CH (CH input channels
// per k-tile): thread -> column n = n0 + tid%128 and channel group
// kr = tid/128 (channels kr*CH/2 .. +CH/2-1 of the tile); the 9 rows of a
// channel are (ki, kj) = (i/3, i%3), i = 0..8, all compile-time.
struct BIm2col3 {
    static constexpr int CH = 2, HC = CH / 2;
    static_assert(CH % 2 == 0, "channel groups split over two thread halves");
    static constexpr int BK = 9 * CH, RB = 9 * HC, PAD = LDP_FWD;
    __amdgpu_buffer_rsrc_t rs;
    int base;      // b*C*H*W + (oh*S-P)*W + (ow*S-P) + kr*H*W
    int HW, W, K, kr;
    unsigned valid; // bit i: (ki,kj) in bounds for this column
    __device__ __forceinline__ void init(const float *x, const ConvGeom &g, int N, int n0,
                                         int tid)
    {
        rs = make_rsrc(x, (unsigned)((size_t)g.B * g.C * g.H * g.W * 4));
        const int n = n0 + tid % GBN;
        kr = tid / GBN;
        HW = g.H * g.W;
        W = g.W;
        K = g.C * 9;
        const int ohw = g.OH * g.OW;
        const bool nok = n < N;
        const int nn = nok ? n : 0;
        const int b = nn / ohw, p = nn - b * ohw;
        const int oh = p / g.OW, ow = p - oh * g.OW;
        const int ihb = oh * g.S - g.P, iwb = ow * g.S - g.P;
        base = b * g.C * HW + ihb * g.W + iwb + kr * HC * HW;
        valid = 0;
#pragma unroll
        for (int i = 0; i < 9; ++i) {
            const int ih = ihb + i / 3, iw = iwb + i % 3;
            if (nok && (unsigned)ih < (unsigned)g.H && (unsigned)iw < (unsigned)g.W)
                valid |= 1u << i;
        }
    }
    __device__ __forceinline__ void load(int k0, int ke, float *rb) const
    {
        // rows k0 + (kr*HC + j)*9 + i belong to channel k0/9 + kr*HC + j
#pragma unroll
        for (int j = 0; j < HC; ++j) {
            const bool cok = k0 + (kr * HC + j) * 9 < ke;
            const int cb = base + (k0 / 9 + j) * HW;
#pragma unroll
            for (int i = 0; i < 9; ++i)
                rb[j * 9 + i] =
                    bload(rs, boff(cok && ((valid >> i) & 1u), cb + (i / 3) * W + (i % 3)));
        }
    }
    template <int LD>
    __device__ __forceinline__ void store(float (*S)[LD], const float *rb) const
    {
        const int nc = ltid() % GBN;
#pragma unroll
        for (int j = 0; j < HC; ++j)
#pragma unroll
            for (int i = 0; i < 9; ++i) S[(kr * HC + j) * 9 + i][nc] = rb[j * 9 + i];
    }
};

// BIm2col3 for inputs with an even channel count (every k-tile full): the
// nine byte offsets of the thread's first channel (out-of-range where the
// tap falls in the padding) are loop-invariant; a k-tile adds the uniform
// (k0/9)*H*W*4 as the scalar offset.  The prefetch after the last tile
// (k0 >= ke) re-reads the last tile.
struct BIm2col3F : BIm2col3 {
    static constexpr bool FULL_K = true;
    unsigned voff[9];
    unsigned hw4;
    __device__ __forceinline__ void init(const float *x, const ConvGeom &g, int N, int n0,
                                         int tid)
    {
        BIm2col3::init(x, g, N, n0, tid);
        hw4 = (unsigned)HW * 4u;
#pragma unroll
        for (int i = 0; i < 9; ++i)
            voff[i] = ((valid >> i) & 1u) ? (unsigned)(base + (i / 3) * W + (i % 3)) * 4u : kOOB;
    }
    __device__ __forceinline__ void load(int k0, int ke, float *rb) const
    {
        static_assert(HC == 1, "one channel per thread group");
        const unsigned d = (unsigned)((k0 < ke ? k0 : k0 - BK) / 9) * hw4;
#pragma unroll
        for (int i = 0; i < 9; ++i) rb[i] = bload_so(rs, voff[i], d);
    }
};

// B for the forward pass with a KS x KS kernel, one input channel per k-tile:
// BK = KS*KS + 1 rows, the last a zero row (KS*KS is odd and a k-step of the
// MFMA takes two rows), so the GEMM runs over a padded K = C*BK.  Thread ->
// column n0 + tid%128 and half kr = tid/128 of the BK rows; the byte offsets
// of its taps (out-of-range for padding taps and the zero row) are
// loop-invariant and a k-tile adds the uniform channel stride.  Used for
// 5x5 (BK = 26); larger kernels would not leave room for two workgroups'
// LDS stages per CU.
template <int KS>
struct BIm2colK {
    static constexpr int T = KS * KS, BK = T + 1, HALF = BK / 2, RB = HALF, PAD = LDP_FWD;
    static_assert(T % 2 == 1, "odd kernel: one zero row completes the k-step");
    __amdgpu_buffer_rsrc_t rs;
    unsigned voff[HALF];
    unsigned hw4;
    int kr;
    __device__ __forceinline__ void init(const float *x, const ConvGeom &g, int N, int n0,
                                         int tid)
    {
        rs = make_rsrc(x, (unsigned)((size_t)g.B * g.C * g.H * g.W * 4));
        const int n = n0 + tid % GBN;
        kr = tid / GBN;
        const int HW = g.H * g.W;
        hw4 = (unsigned)HW * 4u;
        const int ohw = g.OH * g.OW;
        const bool nok = n < N;
        const int nn = nok ? n : 0;
        const int b = nn / ohw, p = nn - b * ohw;
        const int oh = p / g.OW, ow = p - oh * g.OW;
        const int ihb = oh * g.S - g.P, iwb = ow * g.S - g.P;
        const int base = b * g.C * HW + ihb * g.W + iwb;
#pragma unroll
        for (int j = 0; j < HALF; ++j) {
            const int t = kr * HALF + j;
            const int ki = t / KS, kj = t - (t / KS) * KS;
            const bool v = nok && t < T && (unsigned)(ihb + ki) < (unsigned)g.H &&
                           (unsigned)(iwb + kj) < (unsigned)g.W;
            voff[j] = v ? (unsigned)(base + ki * g.W + kj) * 4u : kOOB;
        }
    }
    __device__ __forceinline__ void load(int k0, int ke, float *rb) const
    {
        const unsigned d = (unsigned)((k0 < ke ? k0 : k0 - BK) / BK) * hw4;
#pragma unroll
        for (int j = 0; j < HALF; ++j) rb[j] = bload_so(rs, voff[j], d);
    }
    template <int LD>
    __device__ __forceinline__ void store(float (*S)[LD], const float *rb) const
    {
        const int nc = ltid() % GBN;
#pragma unroll
        for (int j = 0; j < HALF; ++j) S[kr * HALF + j][nc] = rb[j];
    }
};

// The k-major weights for BIm2colK: padded k-tile c covers weight rows
// c*T .. c*T + T-1 and a zero row; float4 loads with loop-invariant offsets.
template <int BM, int KS>
struct AWeightsT4K : AWeightsT4<BM, KS * KS + 1> {
    static constexpr int T = KS * KS, BK = T + 1;
    using Base = AWeightsT4<BM, BK>;
    using Base::NV;
    using Base::C4;
    unsigned voff[NV];
    int TM4;
    __device__ __forceinline__ void init(const float *wt, int M_, int K_, int m0_, int)
    {
        Base::init(wt, M_, K_, m0_, 0);
        TM4 = T * M_ * 4;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int f = ltid() + GNT * i;
            const int row = f / C4, m = m0_ + 4 * (f % C4);
            voff[i] = (f < BK * C4 && row < T && m < M_) ? (unsigned)(row * M_ + m) * 4u : kOOB;
        }
    }
    __device__ __forceinline__ void load(int k0, int ke, float *ra) const
    {
        const unsigned d = (unsigned)((k0 < ke ? k0 : k0 - BK) / BK) * (unsigned)TM4;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const float4 v = bload4_so(this->rs, voff[i], d);
            ra[4 * i] = v.x; ra[4 * i + 1] = v.y; ra[4 * i + 2] = v.z; ra[4 * i + 3] = v.w;
        }
    }
};

// B for the forward pass of a wide KS x KS kernel (KS odd) without padding:
// k-tile t holds two filter rows r = 2t, 2t + 1 of the C*KS rows (channel
// c = r / KS, kernel row ki = r % KS), each as its KS taps and a zero tap,
// BK = 2*(KS + 1); the GEMM runs over K = ceil(C*KS/2) * BK.  Thread ->
// column n0 + tid%128 and row kr = tid/128 of the pair (wave-uniform).  With
// no padding every tap of a valid column lies inside the image, so a
// thread's KS byte offsets are loop-invariant and a k-tile adds the uniform
// (c*H + ki)*W*4 of its row; a row past the last (c >= C) reads zeros.  No
// per-element arithmetic (the generic loader spent about 8 VALU per element
// on the tap's channel, row, column and bounds).
template <int KS>
struct BIm2colRow {
    static constexpr int BK = 2 * (KS + 1), RB = KS + 1, PAD = LDP_FWD;
    static_assert(KS % 2 == 1, "odd kernel: a zero tap completes each row");
    __amdgpu_buffer_rsrc_t rs;
    unsigned voff[KS];
    int kr, C, H, W;
    __device__ __forceinline__ void init(const float *x, const ConvGeom &g, int N, int n0,
                                         int tid)
    {
        rs = make_rsrc(x, (unsigned)((size_t)g.B * g.C * g.H * g.W * 4));
        const int n = n0 + tid % GBN;
        kr = __builtin_amdgcn_readfirstlane(tid / GBN);
        C = g.C;
        H = g.H;
        W = g.W;
        const int ohw = g.OH * g.OW;
        const bool nok = n < N;
        const int nn = nok ? n : 0;
        const int b = nn / ohw, p = nn - b * ohw;
        const int oh = p / g.OW, ow = p - oh * g.OW;
        const int base = b * g.C * g.H * g.W + oh * g.S * g.W + ow * g.S;
#pragma unroll
        for (int j = 0; j < KS; ++j) voff[j] = nok ? (unsigned)(base + j) * 4u : kOOB;
    }
    __device__ __forceinline__ void load(int k0, int, float *rb) const
    {
        const int r = 2 * (k0 / BK) + kr, c = r / KS, ki = r - c * KS;
        const bool rok = c < C;  // uniform: the row exists
        const unsigned d = rok ? (unsigned)((c * H + ki) * W) * 4u : 0u;
#pragma unroll
        for (int j = 0; j < KS; ++j) rb[j] = bload_so(rs, rok ? voff[j] : kOOB, d);
        rb[KS] = 0.f;
    }
    template <int LD>
    __device__ __forceinline__ void store(float (*S)[LD], const float *rb) const
    {
        const int nc = ltid() % GBN;
#pragma unroll
        for (int j = 0; j < RB; ++j) S[kr * RB + j][nc] = rb[j];
    }
};

// The k-major weights Wt[C*KS*KS][M] for BIm2colRow: local row kr*(KS+1) + j
// of k-tile t is weight row (2t + kr)*KS + j (j < KS), or zero for the pad
// tap and for rows past the last; float4 loads with loop-invariant offsets
// and the uniform 2t*KS*M*4 per k-tile.
template <int BM, int KS>
struct AWeightsT4Row : AWeightsT4<BM, 2 * (KS + 1)> {
    static constexpr int BK = 2 * (KS + 1);
    using Base = AWeightsT4<BM, BK>;
    using Base::NV;
    using Base::C4;
    unsigned voff[NV];
    int wrow[NV];  // each float4's weight row at t = 0 (-1: a pad tap)
    int KM4, kw;   // 2*KS*M*4 per k-tile; the weight rows, C*KS*KS
    __device__ __forceinline__ void init_rows(const float *wt, int M_, int kw_, int m0_)
    {
        Base::init(wt, M_, kw_, m0_, 0);
        kw = kw_;
        KM4 = 2 * KS * M_ * 4;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int f = ltid() + GNT * i;
            const int lr = f / C4, m = m0_ + 4 * (f % C4);
            const int half = lr / (KS + 1), j = lr - half * (KS + 1);
            const bool ok = f < BK * C4 && j < KS && m < M_;
            wrow[i] = ok ? half * KS + j : -1;
            voff[i] = ok ? (unsigned)(wrow[i] * M_ + m) * 4u : kOOB;
        }
    }
    __device__ __forceinline__ void load(int k0, int, float *ra) const
    {
        const int t = k0 / BK;
        const unsigned d = (unsigned)t * (unsigned)KM4;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            // rows past the filter's (the second row of a last, odd pair,
            // and the prefetch past the last k-tile) read as zero
            const bool ok = wrow[i] >= 0 && 2 * t * KS + wrow[i] < kw;
            const float4 v = bload4_so(this->rs, ok ? voff[i] : kOOB, ok ? d : 0u);
            ra[4 * i] = v.x; ra[4 * i + 1] = v.y; ra[4 * i + 2] = v.z; ra[4 * i + 3] = v.w;
        }
    }
};

template <class BL> struct RowTaps : std::false_type { static constexpr int ks = 11; };
template <int KS> struct RowTaps<BIm2colRow<KS>> : std::true_type { static constexpr int ks = KS; };

template <class BL> struct PaddedTaps {
    static constexpr bool value = false;
    static constexpr int ks = 5;
};
template <int KS> struct PaddedTaps<BIm2colK<KS>> {
    static constexpr bool value = true;
    static constexpr int ks = KS;
};

// B for the forward pass with any kernel size, BK = 16: thread -> column
// n0 + tid%128, rows tid/128 + 2*i.
template <int KS_T>
struct BIm2colAny {
    static constexpr int BK = 16, RB = 8, PAD = LDP_FWD;
    __amdgpu_buffer_rsrc_t rs;
    int xoff, ihb, iwb, kr, ok, H, W, KS;
    FastDiv dkk, dks;
    __device__ __forceinline__ void init(const float *x, const ConvGeom &g, int N, int n0,
                                         int tid)
    {
        rs = make_rsrc(x, (unsigned)((size_t)g.B * g.C * g.H * g.W * 4));
        const int n = n0 + tid % GBN;
        // the same for the 128 threads of two waves: the rows' (c, ki, kj)
        // are then scalar arithmetic
        kr = __builtin_amdgcn_readfirstlane(tid / GBN);
        ok = n < N;
        H = g.H;
        W = g.W;
        KS = KS_T ? KS_T : g.KS;
        dkk = g.dkk;
        dks = g.dks;
        const int ohw = g.OH * g.OW;
        const int nn = ok ? n : 0;
        const int b = nn / ohw, p = nn - b * ohw;
        const int oh = p / g.OW, ow = p - oh * g.OW;
        xoff = b * g.C * g.H * g.W;
        ihb = oh * g.S - g.P;
        iwb = ow * g.S - g.P;
    }
    __device__ __forceinline__ void load(int k0, int ke, float *rb) const
    {
        const int ks = KS_T ? KS_T : KS, kk2 = ks * ks;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int k = k0 + kr + 2 * i;
            int c, ki;
            if (KS_T) {
                c = k / kk2;
                ki = (k - c * kk2) / ks;
            } else {  // runtime kernel size: magic-number division
                c = fdiv(k, dkk);
                ki = fdiv(k - c * kk2, dks);
            }
            const int t = k - c * kk2, kj = t - ki * ks;
            const int ih = ihb + ki, iw = iwb + kj;
            const bool v = ok && k < ke && (unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W;
            rb[i] = bload(rs, boff(v, xoff + (c * H + ih) * W + iw));
        }
    }
    template <int LD>
    __device__ __forceinline__ void store(float (*S)[LD], const float *rb) const
    {
        const int nc = ltid() % GBN;
#pragma unroll
        for (int i = 0; i < 8; ++i) S[kr + 2 * i][nc] = rb[i];
    }
};


// Weight gradient.  k = b*OHW + p runs over the batch and the output plane.
// A[m][k] = dy[b][m][p]; B[k][n] = x[b][c][oh*S-P+ki][ow*S-P+kj] with
// n = c*KK + ki*KS + kj.  Thread -> k = k0 + tid%BK and rows
// tid/BK + (256/BK)*i; both operands are read in BK-long runs along k, and
// the (c, ki, kj) of a thread's B rows are loop-invariant and precomputed.
struct WgradDivs {
    FastDiv ohw, ow, batch;
};

// LDS rows of the weight-gradient stages are padded to a stride of 2 (mod 32
// floats): a half-wave's transposed stores S[kc][r + RPI*i] (kc = lane % 16,
// r = lane / 16) then hit 32 distinct banks (2*kc + r), and the fragment
// reads (32 consecutive floats of one row) stay conflict-free.
constexpr int WG_PAD = 2;

template <int BM, int BK_>
struct AWgrad {
    static constexpr int BK = BK_, RPI = GNT / BK, RA = BM / RPI, PAD = WG_PAD;
    __amdgpu_buffer_rsrc_t rs;
    int kc, MO;        // MO = M*ohw
    int moff[RA];      // m*ohw or -1
    FastDiv dohw;
    __device__ __forceinline__ void init(const float *dy, const ConvGeom &g, const WgradDivs &dv,
                                         int M, int m0, int tid)
    {
        const int ohw = g.OH * g.OW;
        rs = make_rsrc(dy, (unsigned)((size_t)g.B * M * ohw * 4));
        kc = tid % BK;
        MO = M * ohw;
        dohw = dv.ohw;
#pragma unroll
        for (int i = 0; i < RA; ++i) {
            const int m = m0 + tid / BK + RPI * i;
            moff[i] = m < M ? m * ohw : -1;
        }
    }
    __device__ __forceinline__ void load(int k0, int ke, float *ra) const
    {
        const int k = k0 + kc;
        const bool kok = k < ke;
        const int kk = kok ? k : 0;
        const int b = fdiv(kk, dohw), p = kk - b * (int)dohw.d;
        const int base = b * MO + p;
#pragma unroll
        for (int i = 0; i < RA; ++i) ra[i] = bload(rs, boff(kok && moff[i] >= 0, base + moff[i]));
    }
    template <int LD>
    __device__ __forceinline__ void store(float (*S)[LD], const float *ra) const
    {
        const int r = threadIdx.x / BK;
#pragma unroll
        for (int i = 0; i < RA; ++i) S[kc][r + RPI * i] = ra[i];
    }
};

template <int BN, int BK_, int KS_T>
struct BWgrad {
    static constexpr int BK = BK_, RPI = GNT / BK, RB = BN / RPI, PAD = WG_PAD;
    __amdgpu_buffer_rsrc_t rs;
    int kc, S, P, H, W, CHW;
    FastDiv dohw, dow;
    int coff[RB];      // c*H*W + ki*W + kj, or -1 when n >= N
    int kij[RB];       // ki | kj << 16
    __device__ __forceinline__ void init(const float *x, const ConvGeom &g, const WgradDivs &dv,
                                         int N, int n0, int tid)
    {
        rs = make_rsrc(x, (unsigned)((size_t)g.B * g.C * g.H * g.W * 4));
        kc = tid % BK;
        dohw = dv.ohw;
        dow = dv.ow;
        S = g.S;
        P = g.P;
        H = g.H;
        W = g.W;
        CHW = g.C * g.H * g.W;
        const int ks = KS_T ? KS_T : g.KS, kk2 = ks * ks;
#pragma unroll
        for (int i = 0; i < RB; ++i) {
            const int n = n0 + tid / BK + RPI * i;
            const int c = n / kk2, t = n - c * kk2;
            const int ki = t / ks, kj = t - ki * ks;
            coff[i] = n < N ? c * g.H * g.W + ki * g.W + kj : -1;
            kij[i] = ki | (kj << 16);
        }
    }
    __device__ __forceinline__ void load(int k0, int ke, float *rb) const
    {
        const int k = k0 + kc;
        const bool kok = k < ke;
        const int kk = kok ? k : 0;
        const int b = fdiv(kk, dohw), p = kk - b * (int)dohw.d;
        const int oh = fdiv(p, dow), ow = p - oh * (int)dow.d;
        const int ihb = oh * S - P, iwb = ow * S - P;
        const int base = b * CHW + ihb * W + iwb;
#pragma unroll
        for (int i = 0; i < RB; ++i) {
            const int ih = ihb + (kij[i] & 0xffff), iw = iwb + (kij[i] >> 16);
            const bool v = kok && coff[i] >= 0 && (unsigned)ih < (unsigned)H &&
                           (unsigned)iw < (unsigned)W;
            rb[i] = bload(rs, boff(v, base + coff[i]));
        }
    }
    template <int LD>
    __device__ __forceinline__ void store(float (*S_)[LD], const float *rb) const
    {
        const int r = threadIdx.x / BK;
#pragma unroll
        for (int i = 0; i < RB; ++i) S_[kc][r + RPI * i] = rb[i];
    }
};

// Weight gradient with K reordered as k = (chunk*B + b)*16 + q: position
// p = chunk*16 + q of image b, the plane padded to whole 16-position chunks
// (positions p >= OH*OW read as zero).  A split
// covers images [b0, b1) of ONE position chunk, so each thread's position
// (q = tid % 16), and with it every output row / input tap it reads, is fixed
// for the whole split: the byte offsets are computed once and a k-tile (one
// image) only adds the uniform image stride.  Offsets of invalid elements
// are >= 2^31 and stay out of range after the addition (operands < 2 GiB).
// Both operands are staged K-contiguous (KC: S[row][position], rows of 17
// floats): a thread writes its 16-position run along one row, and a
// fragment's two k-steps are a fixed small offset apart, so the loop reads
// them without address arithmetic.
// Row of element i of thread t when the rows a store instruction writes are
// spread (SPREAD): the four 16-lane groups of a wave take rows 16 apart, so
// at 17 floats per row their 16-bank runs tile the 64 banks (and each
// half-wave's two runs the 32) instead of meeting on a bank, as the four
// consecutive rows of the plain order do.
template <int R>
__device__ __forceinline__ int kc_spread_row(int t, int i)
{
    static_assert(R % 4 == 0, "four rows per thread per 64 rows");
    return (t >> 6) + 4 * (i & 3) + 16 * ((t >> 4) & 3) + 64 * (i >> 2);
}

template <int BM, int BK_, bool SPREAD = false>
struct AWgradC {
    static constexpr int BK = BK_, RPI = GNT / BK, RA = BM / RPI, PAD = WG_PAD;
    // tile row of element i of thread t
    __device__ __forceinline__ static int row(int t, int i)
    {
        if constexpr (SPREAD)
            return kc_spread_row<RA>(t, i);
        else
            return t / BK + RPI * i;
    }
    static constexpr bool KC = true;  // stored as S[m][k]
    static_assert(BK == 16, "one 16-position chunk per k-tile");
    __amdgpu_buffer_rsrc_t rs;
    unsigned voff[RA];
    unsigned img;      // bytes per image of dy
    FastDiv db;
    __device__ __forceinline__ void init(const float *dy, const ConvGeom &g, const WgradDivs &dv,
                                         int M, int m0, int tid, int kb)
    {
        const int ohw = g.OH * g.OW;
        rs = make_rsrc(dy, (unsigned)((size_t)g.B * M * ohw * 4));
        img = (unsigned)(M * ohw) * 4u;
        db = dv.batch;
        const int p = fdiv(kb >> 4, db) * 16 + tid % BK;
#pragma unroll
        for (int i = 0; i < RA; ++i) {
            const int m = m0 + row(tid, i);
            voff[i] = m < M && p < ohw ? (unsigned)(m * ohw + p) * 4u : kOOB;
        }
    }
    __device__ __forceinline__ void load(int k0, int, float *ra) const
    {
        // image (k0/16) mod B: the prefetch past the split wraps to a valid image
        const int t = k0 >> 4;
        const unsigned d = (unsigned)(t - fdiv(t, db) * (int)db.d) * img;
#pragma unroll
        for (int i = 0; i < RA; ++i) ra[i] = bload_so(rs, voff[i], d);
    }
    template <int LD>
    __device__ __forceinline__ void store(float (*S)[LD], const float *ra) const
    {
        const int kc = threadIdx.x % BK;
#pragma unroll
        for (int i = 0; i < RA; ++i) S[row(threadIdx.x, i)][kc] = ra[i];
    }
};

template <int BN, int BK_, int KS_T>
struct BWgradC {
    static constexpr int BK = BK_, RPI = GNT / BK, RB = BN / RPI, PAD = WG_PAD;
    static constexpr bool KC = true;  // stored as S[n][k]
    static_assert(BK == 16, "one 16-position chunk per k-tile");
    __amdgpu_buffer_rsrc_t rs;
    unsigned voff[RB];
    unsigned img;      // bytes per image of x
    FastDiv db;
    __device__ __forceinline__ void init(const float *x, const ConvGeom &g, const WgradDivs &dv,
                                         int N, int n0, int tid, int kb)
    {
        rs = make_rsrc(x, (unsigned)((size_t)g.B * g.C * g.H * g.W * 4));
        img = (unsigned)(g.C * g.H * g.W) * 4u;
        db = dv.batch;
        const int p = fdiv(kb >> 4, db) * 16 + tid % BK;
        const int oh = fdiv(p, dv.ow), ow = p - oh * g.OW;
        const int ihb = oh * g.S - g.P, iwb = ow * g.S - g.P;
        const int ks = KS_T ? KS_T : g.KS, kk2 = ks * ks;
#pragma unroll
        for (int i = 0; i < RB; ++i) {
            const int n = n0 + tid / BK + RPI * i;
            const int c = n / kk2, t = n - c * kk2;
            const int ki = t / ks, kj = t - ki * ks;
            const int ih = ihb + ki, iw = iwb + kj;
            const bool v = n < N && p < g.OH * g.OW && (unsigned)ih < (unsigned)g.H &&
                           (unsigned)iw < (unsigned)g.W;
            voff[i] = v ? (unsigned)((c * g.H + ih) * g.W + iw) * 4u : kOOB;
        }
    }
    __device__ __forceinline__ void load(int k0, int, float *rb) const
    {
        const int t = k0 >> 4;
        const unsigned d = (unsigned)(t - fdiv(t, db) * (int)db.d) * img;
#pragma unroll
        for (int i = 0; i < RB; ++i) rb[i] = bload_so(rs, voff[i], d);
    }
    template <int LD>
    __device__ __forceinline__ void store(float (*S_)[LD], const float *rb) const
    {
        const int r = threadIdx.x / BK, kc = threadIdx.x % BK;
#pragma unroll
        for (int i = 0; i < RB; ++i) S_[r + RPI * i][kc] = rb[i];
    }
};

// ---------------------------------------------------------------------------
// Plain row-major GEMM operands (Gemm.c:116-144), k-tiles of BK_ (16 or 32).
template <bool T, int BR, int BK_ = 16>
struct PlainOperand {
    // element (r, k) of op(X) where X is [R][K] (T = 0) or [K][R] (T = 1);
    // thread map: T = 0 -> k fastest (k = tid%16), T = 1 -> r fastest.
    // Each element's byte offset at k0 = 0 is fixed (rows past R clamped to
    // R-1: they feed only output rows / columns that are never stored); a
    // k-tile adds one uniform offset, and only a k-tile that reaches past
    // the end of its K range tests k per element (zero past the end).
    static constexpr int BK = BK_, RN = BR * BK / GNT, RA = RN, RB = RN, PAD = T ? LDP : 1;
    __amdgpu_buffer_rsrc_t rs;
    int K, ld, r0;
    unsigned voff[RN];
    __device__ __forceinline__ void init(const float *X, int R_, int K_, int ld_, size_t bytes,
                                         int r0_)
    {
        rs = make_rsrc(X, (unsigned)bytes);
        K = K_;
        ld = ld_;
        r0 = r0_;
#pragma unroll
        for (int i = 0; i < RN; ++i) {
            int r, k;
            coords(i, 0, r, k);
            r = r < R_ ? r : R_ - 1;
            voff[i] = (unsigned)(T ? k * ld + r : r * ld + k) * 4u;
        }
    }
    __device__ __forceinline__ void coords(int i, int k0, int &r, int &k) const
    {
        if (!T) { r = r0 + ltid() / BK + (GNT / BK) * i; k = k0 + ltid() % BK; }
        else { r = r0 + ltid() % BR; k = k0 + ltid() / BR + (GNT / BR) * i; }
    }
    __device__ __forceinline__ void load(int k0, int ke, float *v) const
    {
        const unsigned d = (T ? (unsigned)k0 * (unsigned)ld : (unsigned)k0) * 4u;
        if (k0 + BK <= ke) {
#pragma unroll
            for (int i = 0; i < RN; ++i) v[i] = bload_so(rs, voff[i], d);
        } else {
#pragma unroll
            for (int i = 0; i < RN; ++i) {
                int r, k;
                coords(i, k0, r, k);
                v[i] = k < ke ? bload_so(rs, voff[i], d) : 0.f;
            }
        }
    }
    template <int LD>
    __device__ __forceinline__ void store(float (*S)[LD], const float *v) const
    {
#pragma unroll
        for (int i = 0; i < RN; ++i) {
            int r, k;
            coords(i, 0, r, k);
            S[k][r - r0] = v[i];
        }
    }
};

// ===========================================================================
// Problems: operand loaders + k range + epilogue.
// ===========================================================================
// Output epilogue of the forward GEMMs: the layer's bias and activation
// applied to each finished sum, as the separate passes would apply them
// (IOData.addBias then activate, IOData.c:43-72), in one branch-free form
// so the kernel keeps a single epilogue.  Kernels instantiated with the
// epilogue (EPI) hold every accumulator in VGPRs at the end; tiles of at
// most 128 rows keep that within their occupancy.
//   v += bias[m]            (no bias: v + -0.0f, which is v for every v)
//   v = v > 0 ? v : (float)(slope * (double)v)
// slope 0.1 is act_forward's leaky; slope 0 gives relu's v * (v > 0)
// (+-0 with the sign of v, NaN kept); slope 1 is linear.  The default
// (no bias, slope 1) leaves v unchanged.  The logistic activation, with
// its double exp, stays a separate pass.
struct Epi {
    const float *bias = nullptr;
    double slope = 1.0;
    bool active() const { return bias != nullptr || slope != 1.0; }
    __device__ __forceinline__ float apply(float v, int m) const
    {
        const float b = bias ? bias[m] : -0.0f;
        v = v + b;
        return v > 0.f ? v : (float)(slope * (double)v);
    }
};

// Forward: y[b][m][p] = sum_k Wt[k][m] * im2col(x)[k][b*OHW+p].  With
// splits > 1 each z-slice of K writes part[z][m][n] and a fixed-order
// reduction produces y (used when the tile grid alone cannot fill the GPU).
template <int BM_, class BL, bool VECA = false, bool EPI = false>
struct FwdProblem {
    static constexpr int BM = BM_, BN = 128, BK = BL::BK;
    // the next B tile is stored two k-steps before the end of a k-tile
    static constexpr bool EARLY_B = true;
    // the padded-tap loaders end every k-tile with a zero row
    static constexpr bool ODD_K = PaddedTaps<BL>::value;
    // w points at the k-major copy Wt[K][M]; float4 loads when M % 4 == 0
    using AL = typename std::conditional<
        RowTaps<BL>::value, AWeightsT4Row<BM, RowTaps<BL>::ks>,
        typename std::conditional<
            PaddedTaps<BL>::value, AWeightsT4K<BM, PaddedTaps<BL>::ks>,
            typename std::conditional<
                VECA,
                typename std::conditional<std::is_same<BL, BIm2col3F>::value,
                                          AWeightsT4F<BM, BK>, AWeightsT4<BM, BK>>::type,
                AWeightsT<BM, BK>>::type>::type>::type;
    using BLd = BL;
    const float *x, *w;
    float *y, *part;
    ConvGeom g;
    int M, N, K, kchunk, splits;
    Epi e;  // EPI: applied here (only without a K split)
    __device__ __forceinline__ void krange(int z, int &kb, int &ke) const
    {
        kb = z * kchunk;
        ke = min(K, kb + kchunk);
    }
    __device__ __forceinline__ void init_a(AL &a, int m0, int tid, int) const
    {
        if constexpr (RowTaps<BL>::value) a.init_rows(w, M, g.C * g.KS * g.KS, m0);
        else a.init(w, M, K, m0, tid);
    }
    __device__ __forceinline__ void init_b(BL &b, int n0, int tid, int) const { b.init(x, g, N, n0, tid); }
    __device__ __forceinline__ void store(int m, int n, float v, int z) const
    {
        if (m >= M || n >= N) return;
        if (splits > 1) {
            part[((size_t)z * M + m) * N + n] = v;
            return;
        }
        const int ohw = g.OH * g.OW;
        const int b = n / ohw, p = n - b * ohw;
        if constexpr (EPI) v = e.apply(v, m);
        y[((size_t)b * M + m) * ohw + p] = v;
    }
    // The 16 values of one lane of a 32x32 accumulator tile: rows mb +
    // 8*(r/4) + r%4, column n.  The column's image and position (one
    // division) and the base address are computed once per tile, each row
    // is an offset from it.  full: every row of the workgroup's tile is
    // below M (no per-row test).
    __device__ __forceinline__ void store_tile(int mb, int n, const v16f &acc, int z,
                                               bool full) const
    {
        if (n >= N) return;
        float *base;
        int stride;
        if (splits > 1) {
            base = part + ((size_t)z * M + mb) * N + n;
            stride = N;
        } else {
            const int ohw = g.OH * g.OW;
            const int b = n / ohw, p = n - b * ohw;
            base = y + ((size_t)b * M + mb) * ohw + p;
            stride = ohw;
        }
        if (full) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int dm = 8 * (r >> 2) + (r & 3);
                float v = acc[r];
                if constexpr (EPI) v = e.apply(v, mb + dm);
                base[(size_t)dm * stride] = v;
            }
        } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int dm = 8 * (r >> 2) + (r & 3);
                if (mb + dm < M) {
                    float v = acc[r];
                    if constexpr (EPI) v = e.apply(v, mb + dm);
                    base[(size_t)dm * stride] = v;
                }
            }
        }
    }
};

// dW tile stores of the weight-gradient problems (dw[m][n] row-major, one
// lane's 16 values of a 32x32 tile: rows mb + 8*(r/4) + r%4, column n).
// Unsplit: dw += acc with all 16 prior values loaded before the first store;
// with sgd.w the weights are loaded with them and every (w, dw) pair then
// takes the SGD step (sgd_step) on the new dw, so the update costs no pass
// of its own.  Split K: the slice's partial sums.  full: every row of the
// workgroup's tile is below M.
__device__ __forceinline__ void wgrad_store_tile(float *dw, float *part, const Sgd &sgd, int M,
                                                 int N, int splits, int mb, int n,
                                                 const v16f &acc, int z, bool full)
{
    if (n >= N) return;
    if (splits == 1) {
        float *base = dw + (size_t)mb * N + n;
        float old[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int dm = 8 * (r >> 2) + (r & 3);
            old[r] = (full || mb + dm < M) ? base[(size_t)dm * N] : 0.f;
        }
        if (sgd.w) {
            float *wb = sgd.w + (size_t)mb * N + n;
            float wv[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int dm = 8 * (r >> 2) + (r & 3);
                wv[r] = (full || mb + dm < M) ? wb[(size_t)dm * N] : 0.f;
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int dm = 8 * (r >> 2) + (r & 3);
                if (full || mb + dm < M) {
                    float a = wv[r], u = old[r] + acc[r];
                    sgd_step(a, u, sgd.dc, sgd.lc, sgd.mom);
                    wb[(size_t)dm * N] = a;
                    base[(size_t)dm * N] = u;
                }
            }
            return;
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int dm = 8 * (r >> 2) + (r & 3);
            if (full || mb + dm < M) base[(size_t)dm * N] = old[r] + acc[r];
        }
    } else {
        float *base = part + ((size_t)z * M + mb) * N + n;
        if (full) {
#pragma unroll
            for (int r = 0; r < 16; ++r) base[(size_t)(8 * (r >> 2) + (r & 3)) * N] = acc[r];
        } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int dm = 8 * (r >> 2) + (r & 3);
                if (mb + dm < M) base[(size_t)dm * N] = acc[r];
            }
        }
    }
}

template <int BM_, int BN_, int KS_T>
struct WgradProblem {
    static constexpr int BM = BM_, BN = BN_, BK = WGRAD_BK;
    using AL = AWgrad<BM, BK>;
    using BLd = BWgrad<BN, BK, KS_T>;
    const float *x, *dy;
    float *dw, *part;
    ConvGeom g;
    WgradDivs dv;
    int M, N, K, kchunk, splits;
    __device__ __forceinline__ void krange(int z, int &kb, int &ke) const
    {
        kb = z * kchunk;
        ke = min(K, kb + kchunk);
    }
    __device__ __forceinline__ void init_a(AL &a, int m0, int tid, int) const { a.init(dy, g, dv, M, m0, tid); }
    __device__ __forceinline__ void init_b(BLd &b, int n0, int tid, int) const { b.init(x, g, dv, N, n0, tid); }
    // read-modify-write epilogue: prior() of a whole fragment, then store()
    static constexpr bool RMW = true;
    __device__ __forceinline__ float prior(int m, int n, int) const
    {
        return (m < M && n < N && splits == 1) ? dw[(size_t)m * N + n] : 0.f;
    }
    __device__ __forceinline__ void store(int m, int n, float v, float old, int z) const
    {
        if (m >= M || n >= N) return;
        if (splits == 1)
            dw[(size_t)m * N + n] = old + v;
        else
            part[((size_t)z * M + m) * N + n] = v;
    }
};

// Weight gradient in the chunked K order (AWgradC / BWgradC): split z takes
// chunk z / spc and images [(z % spc)*nbs, min(B, (z % spc + 1)*nbs)).
template <int BM_, int BN_, int KS_T>
struct WgradProblemC {
    static constexpr int kWPE = 4;  // waves per SIMD (k_mfma_gemm)
    static constexpr bool EARLY_B = false;  // (k_mfma_gemm's KB_STORE)
    static constexpr int BM = BM_, BN = BN_, BK = WGRAD_BK;
    // the delta operand's stores spread over the banks for the 128 x 96
    // tiles of 3x3 layers (darknet step 6.506-6.513 -> 6.426-6.427 ms and
    // 6.593-6.607 -> 6.523-6.536 ms, three A/B rounds each on two boxes;
    // alone 0.291 -> 0.293 ms).  Spreading AlexNet's tiles too made that
    // step 0.7% slower, and spreading the im2col operand's stores as well
    // (different channels' taps in one load instead of adjacent taps)
    // gained less.
    using AL = AWgradC<BM, BK, BN == 96 && KS_T == 3>;
    using BLd = BWgradC<BN, BK, KS_T>;
    const float *x, *dy;
    float *dw, *part;
    ConvGeom g;
    WgradDivs dv;
    int M, N, spc, nbs, splits;
    Sgd sgd;  // the weights' SGD step in the unsplit epilogue (w == nullptr: none)
    __device__ __forceinline__ void krange(int z, int &kb, int &ke) const
    {
        const int chunk = z / spc, j = z - chunk * spc;
        const int b0 = j * nbs, b1 = min(g.B, b0 + nbs);
        kb = (chunk * g.B + b0) * 16;
        ke = (chunk * g.B + b1) * 16;
    }
    __device__ __forceinline__ void init_a(AL &a, int m0, int tid, int kb) const { a.init(dy, g, dv, M, m0, tid, kb); }
    __device__ __forceinline__ void init_b(BLd &b, int n0, int tid, int kb) const { b.init(x, g, dv, N, n0, tid, kb); }
    // read-modify-write epilogue: prior() of a whole fragment, then store()
    static constexpr bool RMW = true;
    __device__ __forceinline__ float prior(int m, int n, int) const
    {
        return (m < M && n < N && splits == 1) ? dw[(size_t)m * N + n] : 0.f;
    }
    __device__ __forceinline__ void store(int m, int n, float v, float old, int z) const
    {
        if (m >= M || n >= N) return;
        if (splits == 1)
            dw[(size_t)m * N + n] = old + v;
        else
            part[((size_t)z * M + m) * N + n] = v;
    }
    __device__ __forceinline__ void store_tile(int mb, int n, const v16f &acc, int z,
                                               bool full) const
    {
        wgrad_store_tile(dw, part, sgd, M, N, splits, mb, n, acc, z, full);
    }
};

template <bool TA, bool TB>
struct GemmProblem {
    static constexpr int BM = 128, BN = 128, BK = 16;
    using AL = PlainOperand<TA, 128>;
    using BLd = PlainOperand<!TB, 128>;
    const float *A, *Bm;
    float *C;
    int M, N, K, lda, ldb, ldc;
    size_t abytes, bbytes;
    float alpha, beta;
    __device__ __forceinline__ void krange(int, int &kb, int &ke) const { kb = 0; ke = K; }
    __device__ __forceinline__ void init_a(AL &a, int m0, int, int) const { a.init(A, M, K, lda, abytes, m0); }
    __device__ __forceinline__ void init_b(BLd &b, int n0, int, int) const { b.init(Bm, N, K, ldb, bbytes, n0); }
    static constexpr bool RMW = true;
    __device__ __forceinline__ float prior(int m, int n, int) const
    {
        return (m < M && n < N && beta != 0.f) ? C[(size_t)m * ldc + n] : 0.f;
    }
    __device__ __forceinline__ void store(int m, int n, float v, float old, int) const
    {
        if (m >= M || n >= N) return;
        C[(size_t)m * ldc + n] = (beta == 0.f) ? alpha * v : alpha * v + beta * old;
    }
};

// Fully connected layers (a 1x1 convolution of a 1x1 input: x is [B][C],
// y is [B][F], w is [F][C]) as plain GEMMs with coalesced operand loads.
// Forward / input gradient: M = F, N = B, K = C; A = the k-major filter
// Wt[K][M] (m contiguous), B[k][n] = x[n][k] read along k (PlainOperand,
// k fastest); the K split and the output layout are those of FwdProblem.
template <int BM_, bool VECA, bool EPI = false, bool NAT = false, int BK_ = 16>
struct FcProblem {
    static constexpr int BM = BM_, BN = 128, BK = BK_;
    static constexpr bool EARLY_B = true;
    // NAT: w is the filter itself, W[M][K]; else its k-major copy Wt[K][M]
    using AL = typename std::conditional<
        NAT, AWeightsN<BM, BK>,
        typename std::conditional<VECA, AWeightsT4<BM, BK>, AWeightsT<BM, BK>>::type>::type;
    using BLd = PlainOperand<false, 128, BK>;
    const float *x, *w;
    float *y, *part;
    int M, N, K, kchunk, splits;
    size_t xbytes;
    Epi e;
    __device__ __forceinline__ void krange(int z, int &kb, int &ke) const
    {
        kb = z * kchunk;
        ke = min(K, kb + kchunk);
    }
    __device__ __forceinline__ void init_a(AL &a, int m0, int tid, int) const { a.init(w, M, K, m0, tid); }
    __device__ __forceinline__ void init_b(BLd &b, int n0, int, int) const { b.init(x, N, K, K, xbytes, n0); }
    // partial sums take the output's own layout [z][n][m], so the split-K
    // reduction (k_splitk_rows) reads and writes contiguously
    __device__ __forceinline__ void store(int m, int n, float v, int z) const
    {
        if (m >= M || n >= N) return;
        if (splits > 1)
            part[((size_t)z * N + n) * M + m] = v;
        else
            y[(size_t)n * M + m] = EPI ? e.apply(v, m) : v;
    }
};

// Weight gradient of a fully connected layer: M = F, N = C, K = B;
// A[m][k] = dy[k][m] (k-major, m contiguous), B[k][n] = x[k][n] (n
// contiguous, PlainOperand transposed); dw[m][n] += the sum (K split over
// images with a fixed-order reduction when planned).
template <int BM_, bool VECA>
struct FcWgradProblem {
    static constexpr bool EARLY_B = false;  // (k_mfma_gemm's KB_STORE)
    // 4 waves per SIMD (k_mfma_gemm): accumulators in VGPRs, 118-122
    // registers instead of 104 + 64 AGPRs; AlexNet step 7.65 -> 7.57 ms
    static constexpr int kWPE = 4;
    static constexpr int BM = BM_, BN = 128, BK = 16;
    using AL = typename std::conditional<VECA, AWeightsT4<BM, BK>, AWeightsT<BM, BK>>::type;
    using BLd = PlainOperand<true, 128>;
    const float *x, *dy;
    float *dw, *part;
    int M, N, K, kchunk, splits;
    size_t xbytes;
    Sgd sgd;  // the weights' SGD step in the unsplit epilogue (w == nullptr: none)
    __device__ __forceinline__ void krange(int z, int &kb, int &ke) const
    {
        kb = z * kchunk;
        ke = min(K, kb + kchunk);
    }
    __device__ __forceinline__ void init_a(AL &a, int m0, int tid, int) const { a.init(dy, M, K, m0, tid); }
    __device__ __forceinline__ void init_b(BLd &b, int n0, int, int) const { b.init(x, N, K, N, xbytes, n0); }
    __device__ __forceinline__ void store_tile(int mb, int n, const v16f &acc, int z,
                                               bool full) const
    {
        wgrad_store_tile(dw, part, sgd, M, N, splits, mb, n, acc, z, full);
    }
};

// ===========================================================================
template <class P, class = void> struct is_rmw : std::false_type {};
template <class P> struct is_rmw<P, std::void_t<decltype(P::RMW)>> : std::true_type {};
template <class L, class = void> struct kc_layout : std::false_type {};
template <class L> struct kc_layout<L, std::void_t<decltype(L::KC)>> : std::bool_constant<L::KC> {};
template <class P, class = void> struct has_store_tile : std::false_type {};
template <class P>
struct has_store_tile<P, std::void_t<decltype(std::declval<const P &>().store_tile(
                             0, 0, std::declval<const v16f &>(), 0, false))>> : std::true_type {};


// KG > 1: KG groups of GNT threads share one output tile, group g taking
// the K slice z*KG + g of the problem's K split; at the end each group adds
// the other groups' accumulators of the fragments it stores, through LDS.
// With KG = 2 the sum is slice 0 + slice 1, the value a separate reduction
// of the two slices' partials would produce, without writing them.
// Waves per SIMD the compiler must leave room for (P::kWPE, default 1 = no
// constraint).  The weight-gradient problems ask for 4: the compiler then
// keeps the accumulators in ordinary VGPRs (103 registers in all instead of
// 103 VGPRs + 48 AGPRs), so a CU running three of their workgroups keeps
// about 200 registers per SIMD free for the memory-bound kernels of the
// other stream (batch-norm backward reduction: 44 VGPRs, one wave per SIMD
// beside the 152-register waves before); darknet step 6.69 -> 6.64 ms,
// AlexNet 7.69 -> 7.65 ms, the GEMM alone unchanged.
template <class P, class = void> struct odd_last_k : std::false_type {};
template <class P>
struct odd_last_k<P, std::void_t<decltype(P::ODD_K)>> : std::bool_constant<P::ODD_K> {};
template <class P, class = void> struct early_b_store : std::false_type {};
template <class P>
struct early_b_store<P, std::void_t<decltype(P::EARLY_B)>> : std::bool_constant<P::EARLY_B> {};
template <class P, class = void> struct WavesPerEU { static constexpr int v = 1; };
template <class P> struct WavesPerEU<P, std::void_t<decltype(P::kWPE)>> {
    static constexpr int v = P::kWPE;
};
template <class P, int KG = 1>
__global__ void __launch_bounds__(GNT * KG) __attribute__((amdgpu_waves_per_eu(WavesPerEU<P>::v)))
k_mfma_gemm(P p, int mt, int nt)
{
    constexpr int BM = P::BM, BN = P::BN, BK = P::BK;
    static_assert(KG == 1 || KG == 2, "one or two K groups per workgroup");
    // wave grid: 2x2 for 64+ x 128 tiles, 1x4 for 32-row, 4x1 for 32-column
    // and for 128 x 96 tiles (each wave 32 x 96)
    constexpr int WM = BN <= 32 ? 4 : (BN % 64 != 0 && BM % 128 == 0 ? 4 : (BM % 64 == 0 ? 2 : 1));
    constexpr int WN = 4 / WM;
    constexpr int TM = BM / WM / 32, TN = BN / WN / 32;      // MFMA tiles per wave
    // a wave's tiles interleave with the other waves' (rows (i*WM + wm)*32,
    // columns (j*WN + wn)*32): its two fragments of a k-step lie 64 floats
    // apart, which one ds_read2st64 fetches
    static_assert(TM >= 1 && TN >= 1, "tile too small for the wave grid");
    // LDS stages: k-major [BK][rows + PAD], or [rows][BK + 1] for loaders
    // that store a row's K positions contiguously (KC): the odd row length
    // keeps a fragment's 32 rows on 32 banks, and two k-steps of a fragment
    // are a few floats apart (one ds_read2 from a fixed base)
    constexpr bool AKC = kc_layout<typename P::AL>::value, BKC = kc_layout<typename P::BLd>::value;
    constexpr int LA = AKC ? BK + 1 : BM + P::AL::PAD, LB = BKC ? BK + 1 : BN + P::BLd::PAD;
    __shared__ __attribute__((aligned(16))) float Ash[KG][2][AKC ? BM : BK][LA];
    __shared__ __attribute__((aligned(16))) float Bsh[KG][2][BKC ? BN : BK][LB];
    const int grp = KG > 1 ? __builtin_amdgcn_readfirstlane((int)(threadIdx.x / GNT)) : 0;
    auto &As = Ash[grp];
    auto &Bs = Bsh[grp];
    auto rda = [&](int c, int k, int m) -> float {
        if constexpr (AKC) return As[c][m][k];
        else return As[c][k][m];
    };
    auto rdb = [&](int c, int k, int n) -> float {
        if constexpr (BKC) return Bs[c][n][k];
        else return Bs[c][k][n];
    };

    const int tid = (int)threadIdx.x - grp * GNT;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;

    // XCD-aware order over the whole grid: the 8 XCDs take workgroups
    // round-robin in dispatch order (x fastest, then y), so XCD x gets the
    // contiguous range [x*G/8, (x+1)*G/8) of (K slice, tile) pairs, tile
    // fastest and M fastest within it.  The tiles of one K slice then run
    // together on one XCD and read their common operand (the weight-gradient
    // GEMM's delta slice, a forward slice's filter rows) through one L2
    // instead of through all eight.
    const int nblk = mt * nt, total = nblk * (int)gridDim.y;
    int lin = (int)blockIdx.y * nblk + (int)blockIdx.x;
    if ((total & 7) == 0) lin = (lin & 7) * (total >> 3) + (lin >> 3);
    const int z = lin / nblk, tile = lin - z * nblk;
    const int m0 = (tile % mt) * BM, n0 = (tile / mt) * BN;

    int kb, ke;
    p.krange(z * KG + grp, kb, ke);
    typename P::AL al;
    typename P::BLd bl;
    p.init_a(al, m0, tid, kb);
    p.init_b(bl, n0, tid, kb);

    v16f acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    float ra[P::AL::RA], rb[P::BLd::RB];
    int nkt = (ke - kb + BK - 1) / BK;
    if constexpr (KG > 1) {
        // the groups share the barriers, so each runs the longest slice's
        // k-tile count; the host launches KG > 1 only for slices of equal
        // k-tile counts (a group running past its own end would add the
        // re-read last tile of its slice a second time)
#pragma unroll
        for (int q = 0; q < KG; ++q) {
            int qb, qe;
            p.krange(z * KG + q, qb, qe);
            nkt = max(nkt, (qe - qb + BK - 1) / BK);
        }
    }
    if (nkt > 0) {
        al.load(kb, ke, ra);
        bl.load(kb, ke, rb);
        al.template store<LA>(As[0], ra);
        bl.template store<LB>(Bs[0], rb);
    }
    __syncthreads();

    const int lrow = lane >> 5, lcol = lane & 31;
    constexpr int KB_LOAD = BK > 2 ? 2 : 0;  // k-step that issues the B loads
    // k-step that stores the B operand's next tile: two before the last for
    // problems that ask for it (EARLY_B) when the k-tile allows, so the
    // stores complete behind the last MFMAs and the wait before the barrier
    // is short.  The forward / input-gradient and fully connected problems
    // take it (forward probe -1.5%, AlexNet step -0.9%, darknet unchanged);
    // the weight-gradient problems do not: they run beside the critical
    // stream, and faster they made the darknet step 1.3% slower.
    constexpr int KB_STORE = BK >= 8 && early_b_store<P>::value ? BK - 4 : BK - 2;
    // ODD_K problems end every k-tile with a zero row (an odd tap count
    // padded to whole k-steps).  They multiply row by row with two-block
    // MFMAs (v_mfma_f32_32x32x1_2b_f32: two 32x32 outer products, one row of
    // K each), each pairing two fragments that share an operand, which one
    // half of the lanes broadcasts: ODD_COLS pairs a wave's two column
    // fragments (A broadcast, CBSZ 1, ABID = the row's lane half), ODD_ROWS
    // its row fragments 0 and 1 (B broadcast, BLGP 1 / 2).  A k-step of two
    // rows issues as many MFMAs as the 32x32x2 form, and the last one, whose
    // second row is the zero row, half as many (ODD_ROWS: one fewer).  The
    // sums round after every row instead of every pair of rows.
    constexpr bool ODD_COLS = odd_last_k<P>::value && TN == 2;
    constexpr bool ODD_ROWS = odd_last_k<P>::value && TN == 1 && TM >= 2;
    constexpr int NMF_LAST = ODD_COLS ? TM : (ODD_ROWS ? TM - 1 : TM * TN);
    // pairs of accumulator fragments: ODD_COLS (i, 0) and (i, 1) for each i,
    // ODD_ROWS (0, 0) and (1, 0)
    v32f accw[ODD_COLS ? TM : 1];
#pragma unroll
    for (int i = 0; i < (ODD_COLS ? TM : 1); ++i)
#pragma unroll
        for (int r = 0; r < 32; ++r) accw[i][r] = 0.f;
    for (int kt = 0; kt < nkt; ++kt) {
        const int cur = kt & 1;
        // next k-tile (past ke on the last tile: the loaders read zeros or
        // re-read the last tile, and the stores go to the stage nobody reads
        // again)
        const int k0n = kb + (kt + 1) * BK;
        // fragments of k-step kk+2 are read from LDS while the MFMAs of
        // k-step kk issue, so the LDS latency hides behind the matrix pipe
        float a[2][TM], b[2][TN];
        // the broadcast pair operand of rows k and k+1: ODD_COLS the B values
        // of both column fragments, ODD_ROWS the A values of row fragments 0, 1
        float xo[2][2];
        auto read_step = [&](int t, int k) {
            if constexpr (ODD_COLS) {
#pragma unroll
                for (int i = 0; i < TM; ++i) a[t][i] = rda(cur, k + lrow, (i * WM + wm) * 32 + lcol);
                xo[t][0] = rdb(cur, k, (lrow * WN + wn) * 32 + lcol);
                if (k + 2 < BK) xo[t][1] = rdb(cur, k + 1, (lrow * WN + wn) * 32 + lcol);
            } else if constexpr (ODD_ROWS) {
                xo[t][0] = rda(cur, k, (lrow * WM + wm) * 32 + lcol);
                if (k + 2 < BK) xo[t][1] = rda(cur, k + 1, (lrow * WM + wm) * 32 + lcol);
#pragma unroll
                for (int i = 2; i < TM; ++i) a[t][i] = rda(cur, k + lrow, (i * WM + wm) * 32 + lcol);
                b[t][0] = rdb(cur, k + lrow, wn * 32 + lcol);
            } else {
#pragma unroll
                for (int i = 0; i < TM; ++i) a[t][i] = rda(cur, k + lrow, (i * WM + wm) * 32 + lcol);
#pragma unroll
                for (int j = 0; j < TN; ++j) b[t][j] = rdb(cur, k + lrow, (j * WN + wn) * 32 + lcol);
            }
        };
        read_step(0, 0);
#pragma unroll
        for (int kk = 0; kk < BK; kk += 2) {
            const int s = (kk >> 1) & 1;
            if (kk + 2 < BK) read_step(s ^ 1, kk + 2);
            // keep the scheduler from sinking those reads below the MFMAs
            __builtin_amdgcn_sched_barrier(0);
            if (kk == 0) al.load(k0n, ke, ra);
            if (kk == KB_LOAD) bl.load(k0n, ke, rb);
            if constexpr (ODD_COLS) {
#pragma unroll
                for (int i = 0; i < TM; ++i)
                    accw[i] = __builtin_amdgcn_mfma_f32_32x32x1f32(a[s][i], xo[s][0], accw[i], 1, 0, 0);
                if (kk + 2 < BK) {
#pragma unroll
                    for (int i = 0; i < TM; ++i)
                        accw[i] = __builtin_amdgcn_mfma_f32_32x32x1f32(a[s][i], xo[s][1], accw[i], 1, 1,
                                                                       0);
                }
            } else if constexpr (ODD_ROWS) {
                accw[0] = __builtin_amdgcn_mfma_f32_32x32x1f32(xo[s][0], b[s][0], accw[0], 0, 0, 1);
                if (kk + 2 < BK)
                    accw[0] = __builtin_amdgcn_mfma_f32_32x32x1f32(xo[s][1], b[s][0], accw[0], 0, 0, 2);
#pragma unroll
                for (int i = 2; i < TM; ++i)
                    acc[i][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s][i], b[s][0], acc[i][0], 0, 0,
                                                                     0);
            } else {
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s][i], b[s][j], acc[i][j],
                                                                         0, 0, 0);
            }
            if (kk == KB_STORE) bl.template store<LB>(Bs[cur ^ 1], rb);
            if (kk == BK - 2) al.template store<LA>(As[cur ^ 1], ra);
            // interleave: per MFMA one LDS read, a few VALU and one global
            // load (k-steps 0 and 2) or two LDS writes (last k-step)
            // (group masks: 0x008 MFMA, 0x100 DS read, 0x002 VALU,
            //  0x020 VMEM read, 0x200 DS write)
            if (kk == 0 || kk == KB_LOAD) {
#pragma unroll
                for (int t = 0; t < TM * TN; ++t) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
                    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
                }
            } else if (kk == BK - 2 || kk == KB_STORE) {
#pragma unroll
                for (int t = 0; t < (kk == BK - 2 ? NMF_LAST : TM * TN); ++t) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
                    __builtin_amdgcn_sched_group_barrier(0x200, 2, 0);
                }
            }
        }
        __syncthreads();
    }
    if constexpr (ODD_COLS) {
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            acc[i][0] = __builtin_shufflevector(accw[i], accw[i], 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10,
                                                11, 12, 13, 14, 15);
            acc[i][1] = __builtin_shufflevector(accw[i], accw[i], 16, 17, 18, 19, 20, 21, 22, 23, 24,
                                                25, 26, 27, 28, 29, 30, 31);
        }
    } else if constexpr (ODD_ROWS) {
        acc[0][0] = __builtin_shufflevector(accw[0], accw[0], 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11,
                                            12, 13, 14, 15);
        acc[1][0] = __builtin_shufflevector(accw[0], accw[0], 16, 17, 18, 19, 20, 21, 22, 23, 24, 25,
                                            26, 27, 28, 29, 30, 31);
    }

    if constexpr (KG > 1) {
        // group g stores the fragments f = i*TN + j with f % KG == g: it
        // hands the others' fragments over and adds what it receives.  The
        // stages are free after the loop's last barrier: fragments 0 and 1
        // go through the A stages, 2 and 3 through the B stages, each as
        // [register / 4][thread][4]
        static_assert(KG == 2 && TM * TN == 4, "two K groups exchange 4 fragments per wave");
        static_assert(sizeof(Ash) >= 2 * 16 * GNT * sizeof(float) &&
                          sizeof(Bsh) >= 2 * 16 * GNT * sizeof(float),
                      "each stage array holds two exchanged fragments");
        auto xslot = [&](int f, int r4) -> float4 * {
            float4 *base = reinterpret_cast<float4 *>(f < 2 ? &Ash[0][0][0][0] : &Bsh[0][0][0][0]);
            return base + ((f & 1) * 4 + r4) * GNT + tid;
        };
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int f = i * TN + j;
                if (f % KG == grp) continue;
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4)
                    *xslot(f, r4) = make_float4(acc[i][j][4 * r4], acc[i][j][4 * r4 + 1],
                                                acc[i][j][4 * r4 + 2], acc[i][j][4 * r4 + 3]);
            }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int f = i * TN + j;
                if (f % KG != grp) continue;
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4) {
                    const float4 o = *xslot(f, r4);
                    acc[i][j][4 * r4] += o.x;
                    acc[i][j][4 * r4 + 1] += o.y;
                    acc[i][j][4 * r4 + 2] += o.z;
                    acc[i][j][4 * r4 + 3] += o.w;
                }
            }
    }
    // D layout of v_mfma_f32_32x32x2f32: lane l, register r holds
    // row 8*(r/4) + 4*(l/32) + r%4, column l%32.
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            if (KG > 1 && (i * TN + j) % KG != grp) continue;
            const int n = n0 + (j * WN + wn) * 32 + lcol;
            const int mb = m0 + (i * WM + wm) * 32 + 4 * lrow;
            if constexpr (has_store_tile<P>::value) {
                p.store_tile(mb, n, acc[i][j], z, m0 + BM <= p.M);
            } else if constexpr (is_rmw<P>::value) {
                // all 16 prior values in flight before the first store
                float old[16];
#pragma unroll
                for (int r = 0; r < 16; ++r) old[r] = p.prior(mb + 8 * (r >> 2) + (r & 3), n, z);
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    p.store(mb + 8 * (r >> 2) + (r & 3), n, acc[i][j][r], old[r], z);
            } else {
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    p.store(mb + 8 * (r >> 2) + (r & 3), n, acc[i][j][r], z);
            }
        }
}

// ---- forward of a layer with a shallow im2col (K = C*KS*KS <= 32) ---------
// A first layer on an RGB image (3x3: K = 27) has one k-tile of work per
// output tile, so the tiled GEMM above pays its prologue, a padded second
// k-tile and an epilogue that every workgroup reaches at once.  Here each
// wave owns a 32 x 64 output tile and takes its whole K (16 MFMA k-steps,
// K padded to 32 with zeros) straight from global memory into MFMA
// registers: the filter fragments from the k-major copy Wt[K][M], the im2col
// fragments gathered from x with out-of-range taps reading as zero.  No LDS
// and no barrier; 64-column tiles give several waves per SIMD, so one
// wave's output stores overlap another's MFMAs.  WM waves of a workgroup
// split M (32 rows each), 4 / WM split N.  KS_ = 0: kernel size at run time.
template <int WM, int KS_, bool EPI>
__global__ void __launch_bounds__(GNT) k_conv_fwd_smallk(const float *__restrict__ x,
                                                         const float *__restrict__ wt,
                                                         float *__restrict__ y, ConvGeom g,
                                                         FastDiv dohw, FastDiv dow, Epi e)
{
    constexpr int WN = 4 / WM;
    const int KS = KS_ ? KS_ : g.KS, KK = KS * KS;
    const int M = g.F, K = g.C * KK, ohw = (int)dohw.d, N = g.B * ohw;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lrow = lane >> 5, lcol = lane & 31;
    const int wm = wave / WN, wn = wave % WN;
    const int m0 = (blockIdx.y * WM + wm) * 32;
    const int n0 = (blockIdx.x * WN + wn) * 64;
    if (m0 >= M || n0 >= N) return;

    // A: lane holds Wt[2s + lrow][m0 + lcol] for the 16 k-steps s
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(wt, (unsigned)((size_t)M * K * 4));
    const int m = m0 + lcol;
    float a[16];
#pragma unroll
    for (int s = 0; s < 16; ++s) {
        const int k = 2 * s + lrow;
        a[s] = bload(rw, boff(m < M && k < K, k * M + m));
    }
    // B: lane holds im2col(x)[2s + lrow][n0 + 32j + lcol].  The lane's k
    // values are fixed, so their tap offsets (c*H*W + ky*W + kx) and tap
    // coordinates are computed once; per output column only the base
    // address and a validity bit per k-step remain.
    const int HW = g.H * g.W;
    int toff[16];
    int tkyv[16], tkxv[16];
#pragma unroll
    for (int s = 0; s < 16; ++s) {
        const int k = 2 * s + lrow;
        const int c = k / KK, r = k - c * KK, ky = r / KS, kx = r - ky * KS;
        toff[s] = c * HW + ky * g.W + kx;
        tkyv[s] = k < K ? ky : 1 << 20;  // a k past K is never in range
        tkxv[s] = kx;
    }
    const __amdgpu_buffer_rsrc_t rx =
        make_rsrc(x, (unsigned)((size_t)g.B * g.C * HW * 4));
    float b[2][16];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = n0 + 32 * j + lcol;
        const int bi = fdiv(n, dohw), p = n - bi * ohw;
        const int oy = fdiv(p, dow), ox = p - oy * g.OW;
        const int iy0 = oy * g.S - g.P, ix0 = ox * g.S - g.P;
        const int base = bi * g.C * HW + iy0 * g.W + ix0;
        // rows iy0 + ky and columns ix0 + kx inside the image: unsigned
        // compares of the offsets from the image edges
        const unsigned hy = (unsigned)g.H, hx = (unsigned)g.W;
        const bool col_ok = n < N;
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            const bool ok = col_ok && (unsigned)(iy0 + tkyv[s]) < hy &&
                            (unsigned)(ix0 + tkxv[s]) < hx;
            b[j][s] = bload(rx, ok ? (base + toff[s]) * 4 : (int)kOOB);
        }
    }
    v16f acc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[j][r] = 0.f;
#pragma unroll
    for (int s = 0; s < 16; ++s)
#pragma unroll
        for (int j = 0; j < 2; ++j)
            acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s], b[j][s], acc[j], 0, 0, 0);

    // D layout: lane l, register r holds row 8*(r/4) + 4*(l/32) + r%4,
    // column l%32
    const bool full_rows = m0 + 32 <= M;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = n0 + 32 * j + lcol;
        if (n >= N) continue;
        const int bi = fdiv(n, dohw), p = n - bi * ohw;
        float *yb = y + ((size_t)bi * M + m0 + 4 * lrow) * ohw + p;
        if (full_rows) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int mr = m0 + 8 * (r >> 2) + 4 * lrow + (r & 3);
                yb[(size_t)(8 * (r >> 2) + (r & 3)) * ohw] = EPI ? e.apply(acc[j][r], mr) : acc[j][r];
            }
        } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int mr = m0 + 8 * (r >> 2) + 4 * lrow + (r & 3);
                if (mr < M)
                    yb[(size_t)(8 * (r >> 2) + (r & 3)) * ohw] =
                        EPI ? e.apply(acc[j][r], mr) : acc[j][r];
            }
        }
    }
}

// The same with the input patch of the tile staged in LDS.  A workgroup's
// NT = 32*TPW*WN output columns are consecutive positions of one image, which
// read PR input rows (all channels, the full width plus the padding columns)
// into patch[C][PR][PW], zero where the row or column lies outside the image;
// the patch's global loads are all issued before the first LDS write.  Each
// lane's im2col values are then LDS reads at offsets fixed for the lane, with
// no bounds checks.  KST k-steps cover K (14 for 3x3x3).  Each wave owns 32
// filters and TPW tiles of 32 consecutive positions and walks them in order:
// the MFMAs of tile t+1 issue while the stores of tile t drain, so the
// output's HBM writes overlap the matrix work (one tile per MFMA chain, k in
// order, as the single-tile form).  The filter is read as Wt[K][M] or, with
// w_nat, in its own layout W[M][K] (no transposed copy needed).  The host
// takes this kernel when the positions of one image divide into whole tiles
// and the patch fits.
// OWC != 0 (output rows exactly OWC = 32 wide, stride 1, KS_ x KS_): every
// tile is one output row and the patch pitch is OWC + KS_ - 1, so tile t of
// a wave reads t patch rows below tile 0.  The lane's KST LDS addresses are
// then computed once, each tile's reads add only a compile-time offset (no
// address arithmetic or k < K selects per tile), and the k-steps past K
// read a zeroed block after the patch.
template <int WM, int KS_, int KST, bool EPI, int TPW, int OWC = 0>
__global__ void __launch_bounds__(GNT) k_conv_fwd_smallk_lds(const float *__restrict__ x,
                                                             const float *__restrict__ w,
                                                             float *__restrict__ y, ConvGeom g,
                                                             FastDiv dohw, FastDiv dow, Epi e,
                                                             int PR, FastDiv dpw, FastDiv dplane,
                                                             int w_nat)
{
    extern __shared__ float patch[];
    constexpr int WN = 4 / WM, NT = 32 * TPW * WN, U = 8;
    static_assert(OWC == 0 || (OWC == 32 && KS_ > 0), "row tiles need 32-wide rows, fixed KS");
    constexpr int PWC = OWC ? OWC + KS_ - 1 : 0;  // the patch pitch of row tiles
    const int PW = (int)dpw.d;
    const int KS = KS_ ? KS_ : g.KS, KK = KS * KS;
    const int M = g.F, K = g.C * KK, ohw = (int)dohw.d;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lrow = lane >> 5, lcol = lane & 31;
    const int wm = wave / WN, wn = wave % WN;
    const int m0 = (blockIdx.y * WM + wm) * 32;

    // the tile's image and first output row; the patch starts at that row
    const int nt0 = blockIdx.x * NT;
    const int bi = fdiv(nt0, dohw), p0 = nt0 - bi * ohw;
    const int oyf = fdiv(p0, dow);
    const int iyf = oyf * g.S - g.P;
    // the image's planes through a buffer resource: taps outside the image
    // take the out-of-range offset and read as zero
    const __amdgpu_buffer_rsrc_t rx =
        make_rsrc(x + (size_t)bi * g.C * g.H * g.W, (unsigned)(g.C * g.H * g.W) * 4u);
    const int plane = (int)dplane.d, tot = g.C * plane;
    for (int base = 0; base < tot; base += GNT * U) {
        float v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = base + u * GNT + (int)threadIdx.x;
            const int c = fdiv(i, dplane), r0 = i - c * plane, r = fdiv(r0, dpw), q = r0 - r * PW;
            const int iy = iyf + r, ix = q - g.P;
            v[u] = bload(rx, boff(i < tot && iy >= 0 && iy < g.H && ix >= 0 && ix < g.W,
                                  (c * g.H + iy) * g.W + ix));
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = base + u * GNT + (int)threadIdx.x;
            if (i < tot) patch[i] = v[u];
        }
    }
    if constexpr (OWC != 0) {  // the zero block: TPW patch rows
        for (int i = (int)threadIdx.x; i < TPW * PWC; i += GNT) patch[tot + i] = 0.f;
    }
    // A: lane holds W(m0 + lcol, 2s + lrow) for the KST k-steps s
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, (unsigned)((size_t)M * K * 4));
    const int m = m0 + lcol;
    float a[KST];
    int toff[KST];
#pragma unroll
    for (int s = 0; s < KST; ++s) {
        const int k = 2 * s + lrow;
        a[s] = bload(rw, boff(m < M && k < K, w_nat ? m * K + k : k * M + m));
        const int c = k / KK, r = k - c * KK, ky = r / KS, kx = r - ky * KS;
        toff[s] = k < K ? (c * PR + ky) * PW + kx : 0;  // k >= K: read anything, use 0
    }
    __syncthreads();  // the only barrier: waves past it may leave early
    if (m0 >= M) return;

    const int pw0 = p0 + wn * 32 * TPW;  // the wave's first position
    int vb[KST];  // row tiles: the lane's patch index of each k-step in tile 0
    if constexpr (OWC != 0) {
        const int lb0 = (pw0 / OWC - oyf) * PWC + lcol;
#pragma unroll
        for (int s = 0; s < KST; ++s) vb[s] = 2 * s + lrow < K ? lb0 + toff[s] : tot;
    }
    auto fetch = [&](int t, float (&bb)[KST]) {
        if constexpr (OWC != 0) {
#pragma unroll
            for (int s = 0; s < KST; ++s) bb[s] = patch[vb[s] + t * PWC];
            return;
        }
        const int p = pw0 + 32 * t + lcol;
        const int oy = fdiv(p, dow), ox = p - oy * g.OW;
        const int lb = (oy - oyf) * g.S * PW + ox * g.S;
#pragma unroll
        for (int s = 0; s < KST; ++s) {
            const float v = patch[lb + toff[s]];
            bb[s] = 2 * s + lrow < K ? v : 0.f;
        }
    };
    // D layout: lane l, register r holds row 8*(r/4) + 4*(l/32) + r%4,
    // column l%32.  Buffer stores into the wave's rows m0 .. min(m0 + 32, M)
    // - 1 of image bi: the range check of the resource drops the rows past M,
    // each store takes the lane's row offset and the tile's offset (the host
    // keeps 32 rows of a plane below 2^31 bytes).
    const int rows = M - m0 < 32 ? M - m0 : 32;
    const __amdgpu_buffer_rsrc_t ry =
        make_rsrc(y + ((size_t)bi * M + m0) * ohw, (unsigned)(rows * ohw) * 4u);
    unsigned rowv[16];  // the lane's byte offset of each row at the wave's first position
#pragma unroll
    for (int r = 0; r < 16; ++r)
        rowv[r] = (unsigned)((4 * lrow + 8 * (r >> 2) + (r & 3)) * ohw + pw0 + lcol) * 4u;
    float bv[16];  // the rows' biases (rows past M: any valid row, never stored)
    if constexpr (EPI) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int mr = m0 + 8 * (r >> 2) + 4 * lrow + (r & 3);
            bv[r] = e.bias ? e.bias[mr < M ? mr : M - 1] : -0.0f;
        }
    }
    auto val = [&](const v16f &acc, int r) -> float {
        if constexpr (EPI) {  // Epi::apply with the row's bias preloaded
            const float v = acc[r] + bv[r];
            return v > 0.f ? v : (float)(e.slope * (double)v);
        } else {
            return acc[r];
        }
    };
    auto put = [&](int t, const v16f &acc) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(val(acc, r)), ry, (int)rowv[r],
                                                  128 * t, 0);
    };
    float b0[KST], b1[KST];
    v16f acc0, acc1;
    fetch(0, b0);
#pragma unroll
    for (int t = 0; t < TPW; t += 2) {  // TPW even: tiles t (acc0) and t+1 (acc1)
        fetch(t + 1, b1);
#pragma unroll
        for (int r = 0; r < 16; ++r) acc0[r] = 0.f;
#pragma unroll
        for (int s = 0; s < KST; ++s)
            acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s], b0[s], acc0, 0, 0, 0);
        if (t > 0) put(t - 1, acc1);
        if (t + 2 < TPW) fetch(t + 2, b0);
#pragma unroll
        for (int r = 0; r < 16; ++r) acc1[r] = 0.f;
#pragma unroll
        for (int s = 0; s < KST; ++s)
            acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s], b1[s], acc1, 0, 0, 0);
        put(t, acc0);
    }
    put(TPW - 1, acc1);
}

// ---- input gradient of a stride-1 layer with at most 4 input channels ------
// dx[b][c][iy][ix] = sum_f sum_{ky,kx} W[f][c][ky][kx] * dy[b][f][iy+P-ky][ix+P-kx]
// (ConvolutionalLayer.c:931-945 for stride 1).  As a GEMM its M is the
// channel count: a 32-row MFMA tile would compute 29 rows of padding for an
// RGB input, so this runs on the vector ALUs.  A workgroup of DG_WAVES waves
// owns a DG_TH x DG_TW tile of one image; a lane computes 4 adjacent pixels
// of one row for all C channels.  dy is staged in LDS DG_FC filters at a
// time with the tile's halo (zero outside the image), together with those
// filters' weights as wl[f][ky][kx][4 channels], so a lane's tap reads one
// row segment (a float4 and a float2 for 3x3) and one float4 of weights per
// tap for 4*C FMAs.  The next chunk's patch is loaded into registers while
// the current one is computed.  The waves take every DG_WAVES-th filter of
// a chunk and their partial sums are added in wave order through LDS (the
// patch's space), so results do not depend on timing.  The filter is read
// in its own layout W[F][C][KS][KS].
constexpr int DG_TW = 32, DG_TH = 8, DG_FC = 16, DG_WAVES = 8, DG_NT = 64 * DG_WAVES;
// patch rows a wave prefetches per chunk: 4*DG_ROWS, so DG_FC * PH must not
// exceed 4*DG_ROWS*DG_WAVES (kernels up to 9 wide)
constexpr int DG_ROWS = 8;
// 3x3 kernels (the compile-time KS = 3 instance) stage 32 filters per chunk
// (10 prefetched rows per wave): each chunk's compute then covers more of
// the next chunk's load latency, with half as many chunks and barriers
__host__ __device__ constexpr int dg_fc(int ks) { return ks == 3 ? 32 : DG_FC; }
__host__ __device__ constexpr int dg_rows(int ks) { return ks == 3 ? 10 : DG_ROWS; }
template <int NC, int KS_>
__global__ void __launch_bounds__(DG_NT) k_conv_dgrad_smallc(const float *__restrict__ dy,
                                                             const float *__restrict__ w,
                                                             float *__restrict__ dx, ConvGeom g,
                                                             int tiles_x)
{
    extern __shared__ float4 smem4[];
    float *smem = reinterpret_cast<float *>(smem4);
    const int KS = KS_ ? KS_ : g.KS;
    // patch rows padded to a multiple of 4 floats (16-byte aligned segments)
    const int PH = DG_TH + KS - 1, PWd = (DG_TW + KS - 1 + 3) & ~3, pplane = PH * PWd;
    constexpr int FC = dg_fc(KS_), ROWS = dg_rows(KS_);
    float *patch = smem;                                   // [FC][PH][PWd]
    float4 *wl = reinterpret_cast<float4 *>(smem + FC * pplane);  // [FC][KS*KS]
    float *red = smem;  // after the last chunk: [DG_WAVES-1][NC][4][64]
    const int b = blockIdx.y;
    const int tx0 = (blockIdx.x % tiles_x) * DG_TW, ty0 = (blockIdx.x / tiles_x) * DG_TH;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int ty = lane >> 3, tx = (lane & 7) * 4;   // the lane's first pixel in the tile
    // patch row r is dy row oy0 + r, column q is dy column ox0 + q
    const int oy0 = ty0 + g.P - (KS - 1), ox0 = tx0 + g.P - (KS - 1);
    const float *dyb = dy + (size_t)b * g.F * g.OH * g.OW;
    float acc[NC][4];
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[c][q] = 0.f;
    const int taps = KS * KS;
    // slot u of a wave's prefetch holds patch row r = u % PH of the chunk's
    // filter wvu + DG_WAVES * (u / PH), one column per lane: the row's offset
    // is wave-uniform (the loads' scalar operand) and the lane's column
    // offset is fixed, so the loads take no per-slot address registers;
    // columns and rows outside dy read as zero
    constexpr int NU = ROWS * 4;
    const int used = (FC / DG_WAVES) * PH;  // slots in use (host check: <= NU)
    float pre[NU];
    const int wvu = __builtin_amdgcn_readfirstlane(wave);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(dyb, (unsigned)((size_t)g.F * g.OH * g.OW * 4));
    const int oxl = ox0 + lane;
    const unsigned voff = (lane < PWd && oxl >= 0 && oxl < g.OW) ? (unsigned)oxl * 4u : kOOB;
    auto load_chunk = [&](int f0) {
        const int fc = min(FC, g.F - f0);
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            const int fl = wvu + DG_WAVES * (u / PH), oy = oy0 + u % PH;
            const bool ok = u < used && fl < fc && oy >= 0 && oy < g.OH;
            const unsigned soff = ok ? (unsigned)(((f0 + fl) * g.OH + oy) * g.OW) * 4u : 0u;
            pre[u] = bload_so(rs, ok ? voff : kOOB, soff);
        }
    };
    load_chunk(0);
    for (int f0 = 0; f0 < g.F; f0 += FC) {
        const int fc = min(FC, g.F - f0);
        __syncthreads();
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            const int fl = wvu + DG_WAVES * (u / PH);
            if (u < used && lane < PWd) patch[(fl * PH + u % PH) * PWd + lane] = pre[u];
        }
        if constexpr (KS_ == 0) {
            for (int i = threadIdx.x; i < fc * taps; i += DG_NT) {
                const int f = i / taps, tap = i - f * taps;
                const float *wf = w + (size_t)(f0 + f) * NC * taps + tap;
                float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                v.x = wf[0];
                if (NC > 1) v.y = wf[taps];
                if (NC > 2) v.z = wf[2 * taps];
                if (NC > 3) v.w = wf[3 * taps];
                wl[i] = v;
            }
        }
        __syncthreads();
        if (f0 + FC < g.F) load_chunk(f0 + FC);  // in flight while this chunk computes
        for (int f = wvu; f < fc; f += DG_WAVES) {
            const float *pf = patch + f * pplane;
            const float4 *wf = wl + f * taps;
            // compile-time widths read the (wave-uniform) filter's weights
            // straight from W through the scalar cache
            const float *wg = w + (size_t)(f0 + f) * NC * taps;
            for (int ky = 0; ky < KS; ++ky) {
                // row segment: columns tx .. tx + 3 + KS - 1
                const float *row = pf + (ty + KS - 1 - ky) * PWd + tx;
                if constexpr (KS_ != 0) {
                    // compile-time kernel width: the segment in registers
                    float v[4 + KS_ - 1];
                    if constexpr (KS_ == 3) {
                        const float4 v0 = *reinterpret_cast<const float4 *>(row);
                        const float2 v1 = *reinterpret_cast<const float2 *>(row + 4);
                        v[0] = v0.x; v[1] = v0.y; v[2] = v0.z; v[3] = v0.w;
                        v[4] = v1.x; v[5] = v1.y;
                    } else {
#pragma unroll
                        for (int j = 0; j < 4 + KS_ - 1; ++j) v[j] = row[j];
                    }
#pragma unroll
                    for (int kx = 0; kx < KS_; ++kx) {
                        float wc[NC];
#pragma unroll
                        for (int c = 0; c < NC; ++c) wc[c] = wg[c * taps + ky * KS_ + kx];
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const float val = v[q + KS_ - 1 - kx];
#pragma unroll
                            for (int c = 0; c < NC; ++c)
                                acc[c][q] = __fmaf_rn(wc[c], val, acc[c][q]);
                        }
                    }
                } else {
                    // run-time width: each tap value read from LDS (a register
                    // array indexed at run time would live in scratch)
                    for (int kx = 0; kx < KS; ++kx) {
                        const float4 wv = wf[ky * KS + kx];
                        const float wc[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const float val = row[q + KS - 1 - kx];
#pragma unroll
                            for (int c = 0; c < NC; ++c)
                                acc[c][q] = __fmaf_rn(wc[c], val, acc[c][q]);
                        }
                    }
                }
            }
        }
    }
    __syncthreads();  // every wave is done with the last chunk's patch
    if (wave > 0) {
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int q = 0; q < 4; ++q) red[(((wave - 1) * NC + c) * 4 + q) * 64 + lane] = acc[c][q];
    }
    __syncthreads();
    if (wave != 0) return;
    const int iy = ty0 + ty;
    if (iy >= g.H) return;
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int ix = tx0 + tx + q;
            float s = acc[c][q];
            for (int v = 0; v < DG_WAVES - 1; ++v) s += red[((v * NC + c) * 4 + q) * 64 + lane];
            if (ix < g.W) dx[((size_t)(b * NC + c) * g.H + iy) * g.W + ix] = s;
        }
}

// ---- weight gradient of a 1x1 stride-1 layer with few filters -------------
// dW[f][c] += sum over (b, p) of dy[b][f][p] * x[b][c][p]
// (ConvolutionalLayer.c:913-929 for k = 1).  As a GEMM its M is the filter
// count (10 for a classifier's last 1x1 layer) and its K = B*HW is long, so
// the tiled GEMM needs a deep K split and a separate reduction pass.  Here a
// workgroup of WG1_NT threads owns CB channels for every filter and walks
// the whole K in one pass, four positions per float4: thread t takes
// position quads t, t + WG1_NT, ... (x read once; dy read by every
// workgroup, from L2), all of a step's loads in flight together.  Its
// F x CB partial sums are added over the wave (xor tree), then over the
// waves in wave order, and one thread per output adds the total to dW (then
// the weights' SGD step when sg.w is set, as the GEMM epilogues do).  Fixed
// order, no workspace.
constexpr int WG1_NT = 1024;
template <int FMAX, int CB>
__global__ void __launch_bounds__(WG1_NT) k_wgrad_1x1_smallf(const float *__restrict__ x,
                                                             const float *__restrict__ dy,
                                                             float *__restrict__ dw, int B,
                                                             int C, int F, int HW, Sgd sg)
{
    constexpr int NW = WG1_NT / 64;
    __shared__ float red[NW][FMAX * CB];
    const int c0 = blockIdx.x * CB, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float acc[FMAX][CB];
#pragma unroll
    for (int f = 0; f < FMAX; ++f)
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) acc[f][cb] = 0.f;
    const int hw4 = HW >> 2, k4n = B * hw4;
    for (int k4 = threadIdx.x; k4 < k4n; k4 += WG1_NT) {
        const int b = k4 / hw4, p = (k4 - b * hw4) * 4;
        float4 xv[CB], dv[FMAX];
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
            xv[cb] = c0 + cb < C ? *reinterpret_cast<const float4 *>(
                                       x + ((size_t)b * C + c0 + cb) * HW + p)
                                 : make_float4(0.f, 0.f, 0.f, 0.f);
        const float *dyb = dy + (size_t)b * F * HW + p;
#pragma unroll
        for (int f = 0; f < FMAX; ++f)
            dv[f] = f < F ? *reinterpret_cast<const float4 *>(dyb + (size_t)f * HW)
                          : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int f = 0; f < FMAX; ++f)
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) {
                float a = acc[f][cb];
                a = __fmaf_rn(dv[f].x, xv[cb].x, a);
                a = __fmaf_rn(dv[f].y, xv[cb].y, a);
                a = __fmaf_rn(dv[f].z, xv[cb].z, a);
                a = __fmaf_rn(dv[f].w, xv[cb].w, a);
                acc[f][cb] = a;
            }
    }
#pragma unroll
    for (int f = 0; f < FMAX; ++f) {
        if (f < F) {
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) {
                const float v = wave_sum(acc[f][cb]);
                if (lane == 0) red[wave][f * CB + cb] = v;
            }
        }
    }
    __syncthreads();
    const int i = threadIdx.x;
    if (i >= F * CB) return;
    const int f = i / CB, c = c0 + (i - f * CB);
    if (c >= C) return;
    float t = red[0][i];
#pragma unroll
    for (int w = 1; w < NW; ++w) t += red[w][i];
    const size_t o = (size_t)f * C + c;
    float u = dw[o] + t;
    if (sg.w) sgd_step(sg.w[o], u, sg.dc, sg.lc, sg.mom);
    dw[o] = u;
}

__device__ __forceinline__ void addto(float &a, float b) { a += b; }
__device__ __forceinline__ void addto(float4 &a, const float4 &b)
{
    a.x += b.x;
    a.y += b.y;
    a.z += b.z;
    a.w += b.w;
}

// sum of part[z][i] over z in [z0, z1), in z order from 0: eight slices'
// loads are issued before their (in-order) adds
template <class T>
__device__ __forceinline__ T slice_sum(const T *__restrict__ p, size_t n, size_t i, int z0, int z1)
{
    T s;
    if constexpr (std::is_same<T, float4>::value) s = make_float4(0.f, 0.f, 0.f, 0.f);
    else s = 0.f;
    int z = z0;
    for (; z + 8 <= z1; z += 8) {
        T v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = p[(size_t)(z + u) * n + i];
#pragma unroll
        for (int u = 0; u < 8; ++u) addto(s, v[u]);
    }
    for (; z < z1; ++z) addto(s, p[(size_t)z * n + i]);
    return s;
}

// Fixed-order split-K reduction: dw[i] += sum_z part[z][i], z ascending.
// V4: four consecutive outputs per thread as float4 (mn % 4 == 0, 16-byte
// aligned operands); the same additions in the same order.  With sg.w the
// weights' SGD step (sgd_step) follows on each (w[i], dw[i]) in the same
// pass, the values of ach_sgd_update over dw afterwards.
template <bool V4>
__global__ void __launch_bounds__(256) k_splitk_reduce(const float *__restrict__ part,
                                                       float *__restrict__ dw, size_t mn,
                                                       int splits, Sgd sg)
{
    typedef typename std::conditional<V4, float4, float>::type T;
    const size_t n = V4 ? mn / 4 : mn;
    const T *p = reinterpret_cast<const T *>(part);
    T *d = reinterpret_cast<T *>(dw);
    T *w = reinterpret_cast<T *>(sg.w);
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        const T s = slice_sum(p, n, i, 0, splits);
        T o = d[i];
        addto(o, s);
        if (w) {
            T a = w[i];
            if constexpr (V4) {
                sgd_step(a.x, o.x, sg.dc, sg.lc, sg.mom);
                sgd_step(a.y, o.y, sg.dc, sg.lc, sg.mom);
                sgd_step(a.z, o.z, sg.dc, sg.lc, sg.mom);
                sgd_step(a.w, o.w, sg.dc, sg.lc, sg.mom);
            } else {
                sgd_step(a, o, sg.dc, sg.lc, sg.mom);
            }
            w[i] = a;
        }
        d[i] = o;
    }
}

// First level for many splits: tmp[c][i] = sum of part[z][i] over the
// SPLIT_GROUP consecutive z of group c (z ascending); the second level is
// k_splitk_reduce over the groups.  Keeps every output's sum order fixed.
constexpr int SPLIT_GROUP = 32;
template <bool V4>
__global__ void __launch_bounds__(256) k_splitk_group(const float *__restrict__ part,
                                                      float *__restrict__ tmp, size_t mn,
                                                      int splits)
{
    typedef typename std::conditional<V4, float4, float>::type T;
    const size_t n = V4 ? mn / 4 : mn;
    const T *p = reinterpret_cast<const T *>(part);
    T *t = reinterpret_cast<T *>(tmp);
    const int c = blockIdx.y;
    const int z0 = c * SPLIT_GROUP, z1 = min(splits, z0 + SPLIT_GROUP);
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        t[(size_t)c * n + i] = slice_sum(p, n, i, z0, z1);
}

// Wt[k][m] = W[m][k]: the k-major copy of the filter the forward GEMM reads
// (32x32 tiles through LDS so both sides stay coalesced).
__global__ void __launch_bounds__(256) k_weights_kmajor(const float *__restrict__ w,
                                                        float *__restrict__ wt, int M, int K)
{
    __shared__ float t[32][33];
    const int k0 = blockIdx.x * 32, m0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int r = ty; r < 32; r += 8) {
        const int m = m0 + r, k = k0 + tx;
        t[r][tx] = (m < M && k < K) ? w[(size_t)m * K + k] : 0.f;
    }
    __syncthreads();
    for (int r = ty; r < 32; r += 8) {
        const int k = k0 + r, m = m0 + tx;
        if (k < K && m < M) wt[(size_t)k * M + m] = t[tx][r];
    }
}

// Flipped, transposed filter for stride-1 dgrad, k-major:
// Wft[(f*KK + t)*C + c] = W[f][c][KK-1-t], i.e. the forward filter of a
// convolution of dy (F input channels) producing C channels with pad k-1-p.
__global__ void k_weights_flip_kmajor(const float *__restrict__ w, float *__restrict__ wft,
                                      int F, int C, int KK)
{
    const size_t total = (size_t)F * C * KK;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const int c = (int)(i % C);
        const size_t ft = i / C;
        const int t = (int)(ft % KK);
        const int f = (int)(ft / KK);
        wft[i] = w[((size_t)f * C + c) * KK + (KK - 1 - t)];
    }
}

// Batched filter preparation: for every job one launch writes the k-major
// copy Wt[K][M] (32x32 LDS tiles) and, when asked, the flipped k-major copy
// Wft[(f*KK + t)*C + c] = W[f][c][KK-1-t] (one thread per filter channel).
constexpr int PREP_MAX_JOBS = 32;
struct PrepJob {
    const float *w;
    float *wt, *wft;
    int M, C, KK;     // filters, input channels, taps
    int tiles_t;      // k-major transpose tiles: ceil(K/32) * ceil(M/32)
    int tiles_f;      // flip blocks: ceil(M*C/256), 0 when no flipped copy
};
struct PrepTable {
    PrepJob job[PREP_MAX_JOBS];
    int n;
};

__global__ void __launch_bounds__(256) k_prepare_filters(PrepTable tab)
{
    __shared__ float t[32][33];
    int b = blockIdx.x, j = 0;
    while (j < tab.n && b >= tab.job[j].tiles_t + tab.job[j].tiles_f) {
        b -= tab.job[j].tiles_t + tab.job[j].tiles_f;
        ++j;
    }
    if (j >= tab.n) return;
    const PrepJob &J = tab.job[j];
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    if (b < J.tiles_t) {
        const int K = J.C * J.KK, M = J.M;
        const int kt = (K + 31) / 32;
        const int k0 = (b % kt) * 32, m0 = (b / kt) * 32;
        for (int r = ty; r < 32; r += 8) {
            const int m = m0 + r, k = k0 + tx;
            t[r][tx] = (m < M && k < K) ? J.w[(size_t)m * K + k] : 0.f;
        }
        __syncthreads();
        for (int r = ty; r < 32; r += 8) {
            const int k = k0 + r, m = m0 + tx;
            if (k < K && m < M) J.wt[(size_t)k * M + m] = t[tx][r];
        }
        return;
    }
    // flip: one thread per (filter, channel) copies its KK taps; neighbouring
    // threads read adjacent tap runs and write adjacent channels of a tap.
    // 3x3 (and 5x5) filters load all their taps before the first store.
    const int fc = (b - J.tiles_t) * 256 + threadIdx.x;
    if (fc >= J.M * J.C) return;
    const int f = fc / J.C, c = fc - f * J.C, KK = J.KK;
    const float *src = J.w + (size_t)fc * KK;
    float *dst = J.wft + (size_t)f * KK * J.C + c;
    auto flip = [&](auto kk) {
        constexpr int T = decltype(kk)::value;
        float v[T];
#pragma unroll
        for (int tap = 0; tap < T; ++tap) v[tap] = src[T - 1 - tap];
#pragma unroll
        for (int tap = 0; tap < T; ++tap) dst[(size_t)tap * J.C] = v[tap];
    };
    if (KK == 9) flip(std::integral_constant<int, 9>());
    else if (KK == 25) flip(std::integral_constant<int, 25>());
    else
        for (int tap = 0; tap < KK; ++tap) dst[(size_t)tap * J.C] = src[KK - 1 - tap];
}

// ---------------------------------------------------------------------------
// splits: the problem's K slices; KG of them share a workgroup
template <class P, int KG = 1>
static int launch_gemm(const P &p, int M, int N, int splits, hipStream_t st)
{
    const int mt = (M + P::BM - 1) / P::BM, nt = (N + P::BN - 1) / P::BN;
    if ((long long)mt * nt * splits > 0x7fffffffLL || splits > 65535 || splits % KG != 0)
        return ACH_EINVAL;
    hipLaunchKernelGGL((k_mfma_gemm<P, KG>), dim3(mt * nt, splits / KG), dim3(GNT * KG), 0, st, p,
                       mt, nt);
    return check_launch();
}

static bool conv_ok(const ach_conv_desc *d)
{
    return d && d->batch > 0 && d->c > 0 && d->h > 0 && d->w > 0 && d->n > 0 &&
           d->size > 0 && d->stride > 0 && d->stride_y >= 0 && d->pad >= 0 &&
           (d->h + 2 * d->pad - d->size) >= 0 && (d->w + 2 * d->pad - d->size) >= 0;
}

// height stride (stride_y 0: the width stride)
static int stride_h(const ach_conv_desc *d) { return d->stride_y > 0 ? d->stride_y : d->stride; }

static ConvGeom geom(const ach_conv_desc *d)
{
    ConvGeom g;
    g.B = d->batch; g.C = d->c; g.H = d->h; g.W = d->w;
    g.F = d->n; g.KS = d->size; g.S = d->stride; g.P = d->pad;
    g.OH = (d->h + 2 * d->pad - d->size) / stride_h(d) + 1;
    g.OW = (d->w + 2 * d->pad - d->size) / d->stride + 1;
    // A kernel that covers the whole unpadded input (one output position: the
    // fully connected layers expressed as convolutions) is a 1x1 convolution
    // of the flattened input [B][C*k*k][1][1]; x, w, y, dx and dw keep their
    // memory layout and the k order (c, ki, kj) is the same.
    if (g.OH == 1 && g.OW == 1 && g.P == 0 && g.KS == g.H && g.KS == g.W && g.KS > 1) {
        g.C = g.C * g.KS * g.KS;
        g.H = g.W = 1;
        g.KS = 1;
        g.S = 1;
    }
    g.dkk = make_fastdiv((unsigned)(g.KS * g.KS));
    g.dks = make_fastdiv((unsigned)g.KS);
    return g;
}

// Buffer loads address bytes with 32-bit offsets: every operand must stay
// below 2 GiB.
static bool fits_int(const ach_conv_desc *d)
{
    const ConvGeom g = geom(d);
    const double lim = 536870911.0;  // floats in 2 GiB - 4 bytes
    const double in = (double)g.B * g.C * g.H * g.W;
    const double out = (double)g.B * g.F * g.OH * g.OW;
    return in <= lim && out <= lim && (double)g.F * g.C * g.KS * g.KS <= lim;
}

// ---- unequal width / height strides ----------------------------------------
// The reference's per-image passes (ConvolutionalLayer.c:790-803, 913-945),
// each image's im2col, GEMM and col2im a device launch of ach_im2col /
// ach_gemm / ach_col2im over one image's column buffer [C*k*k][OH*OW] in
// the workspace.  The tiled implicit-GEMM loaders take one stride; a fully
// connected geometry (one output position) is unaffected by the strides and
// keeps its own path.
static bool fc_geom(const ConvGeom &g);
static bool conv_xy(const ach_conv_desc *d)
{
    return stride_h(d) != d->stride && !fc_geom(geom(d));
}

static size_t xy_col_bytes(const ConvGeom &g)
{
    return (size_t)g.C * g.KS * g.KS * g.OH * g.OW * sizeof(float);
}

// y_b = W * im2col(x_b); w is [F][K], or k-major [K][F] when kmajor
static int xy_fwd(const ach_conv_desc *d, const float *x, const float *w, bool kmajor, float *y,
                  void *ws, size_t ws_bytes, ach_stream_t st)
{
    const ConvGeom g = geom(d);
    if (!ws || ws_bytes < xy_col_bytes(g)) return ACH_EWORKSPACE;
    const int m = g.F, k = g.C * g.KS * g.KS, n = g.OH * g.OW;
    float *col = (float *)ws;
    for (int i = 0; i < g.B; ++i) {
        int rc = ach_im2col(x + (size_t)i * g.C * g.H * g.W, g.C, g.H, g.W, g.KS, g.KS, g.P, g.P,
                            stride_h(d), d->stride, 1, 1, col, st);
        if (rc) return rc;
        rc = kmajor ? ach_gemm(1, 0, m, n, k, 1.f, w, m, col, n, 0.f, y + (size_t)i * m * n, n, st)
                    : ach_gemm(0, 0, m, n, k, 1.f, w, k, col, n, 0.f, y + (size_t)i * m * n, n, st);
        if (rc) return rc;
    }
    return ACH_OK;
}

// dw += dy_b * im2col(x_b)^T over the images in order
static int xy_bwd_filter(const ach_conv_desc *d, const float *x, const float *dy, float *dw,
                         void *ws, size_t ws_bytes, ach_stream_t st)
{
    const ConvGeom g = geom(d);
    if (!ws || ws_bytes < xy_col_bytes(g)) return ACH_EWORKSPACE;
    const int m = g.F, n = g.C * g.KS * g.KS, k = g.OH * g.OW;
    float *col = (float *)ws;
    for (int i = 0; i < g.B; ++i) {
        int rc = ach_im2col(x + (size_t)i * g.C * g.H * g.W, g.C, g.H, g.W, g.KS, g.KS, g.P, g.P,
                            stride_h(d), d->stride, 1, 1, col, st);
        if (rc) return rc;
        rc = ach_gemm(0, 1, m, n, k, 1.f, dy + (size_t)i * m * k, k, col, k, 1.f, dw, n, st);
        if (rc) return rc;
    }
    return ACH_OK;
}

// y[b][m][p] = sum_z part[z][m][b*OHW+p], z ascending (fixed order), then
// the epilogue.  V4: four consecutive positions of one plane per thread as
// float4 (OHW % 4 == 0, 16-byte aligned operands); the same additions.
template <bool EPI, bool V4>
__global__ void __launch_bounds__(256) k_splitk_to_nchw(const float *__restrict__ part,
                                                        float *__restrict__ y, int M, int N,
                                                        FastDiv dohw, FastDiv dM, int splits,
                                                        Epi e)
{
    // M*N < 2^29 (operands below 2 GiB): 32-bit indices, magic-number division
    constexpr int V = V4 ? 4 : 1;
    typedef typename std::conditional<V4, float4, float>::type T;
    const int mn = M * N, ohw = (int)dohw.d;
    const T *pt = reinterpret_cast<const T *>(part);
    for (int q = blockIdx.x * blockDim.x + threadIdx.x; q < mn / V;
         q += gridDim.x * blockDim.x) {
        const int i = q * V;
        const int bm = fdiv(i, dohw), p = i - bm * ohw;
        const int b = fdiv(bm, dM), m = bm - b * M;
        const int n = b * ohw + p;
        T s = slice_sum(pt, (size_t)mn / V, (size_t)(m * N + n) / V, 0, splits);
        if constexpr (V4) {
            if constexpr (EPI) {
                s.x = e.apply(s.x, m);
                s.y = e.apply(s.y, m);
                s.z = e.apply(s.z, m);
                s.w = e.apply(s.w, m);
            }
            reinterpret_cast<float4 *>(y)[q] = s;
        } else {
            y[i] = EPI ? e.apply(s, m) : s;
        }
    }
}

// The same reduction walked in the partials' order for planes whose size is
// not a multiple of 4 (N % 4 == 0, 16-byte aligned part): four consecutive
// n of one filter row per thread, loaded as float4, summed in the same
// order, stored one by one (they may cross an image boundary).
template <bool EPI>
__global__ void __launch_bounds__(256) k_splitk_to_nchw_pv(const float *__restrict__ part,
                                                           float *__restrict__ y, int M, int N,
                                                           FastDiv dohw, FastDiv dN, int splits,
                                                           Epi e)
{
    const int mn = M * N, ohw = (int)dohw.d;
    const float4 *pt = reinterpret_cast<const float4 *>(part);
    for (int q = blockIdx.x * blockDim.x + threadIdx.x; q < mn / 4;
         q += gridDim.x * blockDim.x) {
        const int i = q * 4;
        const int m = fdiv(i, dN), n = i - m * N;
        int b = fdiv(n, dohw), pp = n - b * ohw;
        const float4 s = slice_sum(pt, (size_t)mn / 4, (size_t)q, 0, splits);
        const float v[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            y[((size_t)b * M + m) * ohw + pp] = EPI ? e.apply(v[j], m) : v[j];
            if (++pp == ohw) { pp = 0; ++b; }
        }
    }
}

// The same reduction for partials already in the output's layout (the
// fully connected GEMMs): y[i] = sum_z part[z][i], z ascending, then the
// epilogue with m = i mod M.  V4 as above (mn % 4 == 0).
template <bool EPI, bool V4>
__global__ void __launch_bounds__(256) k_splitk_rows(const float *__restrict__ part,
                                                     float *__restrict__ y, int mn, FastDiv dM,
                                                     int splits, Epi e)
{
    constexpr int V = V4 ? 4 : 1;
    typedef typename std::conditional<V4, float4, float>::type T;
    const T *pt = reinterpret_cast<const T *>(part);
    for (int q = blockIdx.x * blockDim.x + threadIdx.x; q < mn / V;
         q += gridDim.x * blockDim.x) {
        T s = slice_sum(pt, (size_t)mn / V, (size_t)q, 0, splits);
        if constexpr (V4) {
            if constexpr (EPI) {
                const int M = (int)dM.d;
                int m = 4 * q - fdiv(4 * q, dM) * M;
                s.x = e.apply(s.x, m);
                m = m + 1 == M ? 0 : m + 1;
                s.y = e.apply(s.y, m);
                m = m + 1 == M ? 0 : m + 1;
                s.z = e.apply(s.z, m);
                m = m + 1 == M ? 0 : m + 1;
                s.w = e.apply(s.w, m);
            }
            reinterpret_cast<float4 *>(y)[q] = s;
        } else {
            if constexpr (EPI) s = e.apply(s, q - fdiv(q, dM) * (int)dM.d);
            y[q] = s;
        }
    }
}

// Forward tiling plan: BM from the filter count; K split into `splits`
// slices (a multiple of the k-tile each) when the tile grid alone gives
// fewer than ~2 workgroups per CU.  Depends only on the shape, so results are
// reproducible run to run.
struct FwdPlan {
    int bm, bk, splits, kchunk;
    int kg;  // K slices per workgroup (kg == splits: no partial sums)
    // partial-sum slices written (each workgroup adds its kg slices first)
    int pslices() const { return splits / kg; }
};

// a 1x1 convolution of a 1x1 input (the fully connected layers once geom()
// has flattened them): FcProblem / FcWgradProblem
static bool fc_geom(const ConvGeom &g) { return g.KS == 1 && g.H == 1 && g.W == 1 && g.P == 0; }
// k-tile of the fully connected GEMMs with 128-row tiles: their grids give
// one 8-wave workgroup per CU (two waves per SIMD), too few to hide the
// operand loads behind one 16-wide k-tile of MFMAs
constexpr int FC_BK = 32;

// 5x5 filters with a filter count divisible by 4 take the padded-tap
// loaders (BIm2colK<5> / AWeightsT4K)
static bool fwd_padded_taps(const ConvGeom &g) { return g.KS == 5 && (g.F & 3) == 0; }
// 11x11 filters without padding (AlexNet's first layer), a filter count
// divisible by 4: the row-tap loaders (k-tiles of two filter rows)
constexpr int ROW_KS = 11;
static bool fwd_row_taps(const ConvGeom &g)
{
    return g.KS == ROW_KS && g.P == 0 && (g.F & 3) == 0 && !fc_geom(g);
}
static int fwd_row_k(const ConvGeom &g)
{
    return (g.C * g.KS + 1) / 2 * BIm2colRow<ROW_KS>::BK;
}

// the shallow-im2col forward (k_conv_fwd_smallk) takes these geometries
static bool fwd_small_k(const ConvGeom &g)
{
    return !fc_geom(g) && g.C * g.KS * g.KS <= 32;
}

template <int WM, int KS, bool EPI>
static int smallk_launch(const ConvGeom &g, const float *x, const float *wt, float *y,
                         const Epi &e, hipStream_t st)
{
    const int N = g.B * g.OH * g.OW;
    const dim3 grid((N + 64 * (4 / WM) - 1) / (64 * (4 / WM)), (g.F + 32 * WM - 1) / (32 * WM));
    if (grid.y > 65535) return ACH_EUNSUPPORTED;
    hipLaunchKernelGGL((k_conv_fwd_smallk<WM, KS, EPI>), grid, dim3(GNT), 0, st, x, wt, y, g,
                       make_fastdiv((unsigned)(g.OH * g.OW)), make_fastdiv((unsigned)g.OW), e);
    return check_launch();
}

// the patch-staged kernel: returns ACH_EUNSUPPORTED when its conditions fail.
// Tiles per wave: the most of 8, 4, 2 whose workgroup span divides the
// positions of an image and still leaves 512 workgroups (fewer tiles per
// wave when the grid would not fill the GPU twice over).
template <int WM, int KS, int KST, bool EPI, int TPW, int OWC>
static int smallk_lds_go(const ConvGeom &g, const float *x, const float *w, float *y,
                         const Epi &e, bool w_nat, hipStream_t st)
{
    constexpr int NT = 32 * TPW * (4 / WM);
    const int N = g.B * g.OH * g.OW, ohw = g.OH * g.OW;
    const dim3 grid(N / NT, (g.F + 32 * WM - 1) / (32 * WM));
    // the input rows of the output rows a tile spans
    const int rows = (NT + g.OW - 2) / g.OW + 1;
    const int PR = (rows - 1) * g.S + g.KS, PW = g.W + 2 * g.P;
    // row tiles add a zero block of TPW patch rows
    const size_t lds = ((size_t)g.C * PR * PW + (OWC ? (size_t)TPW * PW : 0)) * sizeof(float);
    if (ohw % NT != 0 || lds > 32768 || grid.y > 65535 || (size_t)ohw * 32 * 4 >= (1u << 31))
        return ACH_EUNSUPPORTED;
    if (OWC && (g.OW != OWC || g.S != 1 || g.KS != KS || PW != OWC + KS - 1))
        return ACH_EUNSUPPORTED;
    hipLaunchKernelGGL((k_conv_fwd_smallk_lds<WM, KS, KST, EPI, TPW, OWC>), grid, dim3(GNT), lds,
                       st,
                       x, w, y, g, make_fastdiv((unsigned)ohw), make_fastdiv((unsigned)g.OW), e,
                       PR, make_fastdiv((unsigned)PW), make_fastdiv((unsigned)(PR * PW)),
                       (int)w_nat);
    return check_launch();
}

template <int WM, int KS, int KST, bool EPI, int OWC = 0>
static int smallk_lds_launch(const ConvGeom &g, const float *x, const float *w, float *y,
                             const Epi &e, bool w_nat, hipStream_t st)
{
    constexpr int WN = 4 / WM;
    const long long N = (long long)g.B * g.OH * g.OW;
    const long long fb = (g.F + 32 * WM - 1) / (32 * WM);
    if (N / (32 * 8 * WN) * fb >= 512) {
        const int rc = smallk_lds_go<WM, KS, KST, EPI, 8, OWC>(g, x, w, y, e, w_nat, st);
        if (rc != ACH_EUNSUPPORTED) return rc;
    }
    if (N / (32 * 4 * WN) * fb >= 512) {
        const int rc = smallk_lds_go<WM, KS, KST, EPI, 4, OWC>(g, x, w, y, e, w_nat, st);
        if (rc != ACH_EUNSUPPORTED) return rc;
    }
    return smallk_lds_go<WM, KS, KST, EPI, 2, OWC>(g, x, w, y, e, w_nat, st);
}

template <int WM, bool EPI>
static int smallk_lds_ks(const ConvGeom &g, const float *x, const float *w, float *y,
                         const Epi &e, bool w_nat, hipStream_t st)
{
    // 3x3 over 3 channels (K = 27): 14 k-steps, in row tiles for 32-wide
    // stride-1 outputs; otherwise the full 16
    if (g.KS == 3 && g.C == 3 && g.OW == 32 && g.S == 1) {
        const int rc = smallk_lds_launch<WM, 3, 14, EPI, 32>(g, x, w, y, e, w_nat, st);
        if (rc != ACH_EUNSUPPORTED) return rc;
    }
    if (g.KS == 3 && g.C == 3) return smallk_lds_launch<WM, 3, 14, EPI>(g, x, w, y, e, w_nat, st);
    if (g.KS == 3) return smallk_lds_launch<WM, 3, 16, EPI>(g, x, w, y, e, w_nat, st);
    return smallk_lds_launch<WM, 0, 16, EPI>(g, x, w, y, e, w_nat, st);
}

// w: Wt[K][M], or W[M][K] with w_nat (the patch-staged kernel reads either;
// the register-gather fallback needs Wt and returns ACH_EUNSUPPORTED for w_nat)
template <bool EPI>
static int fwd_small_k_launch(const ConvGeom &g, const float *x, const float *w, float *y,
                              const Epi &e, bool w_nat, hipStream_t st)
{
    // waves along M: 4 for more than 64 filters, 2 for 33-64, 1 for <= 32
    int rc = g.F > 64 ? smallk_lds_ks<4, EPI>(g, x, w, y, e, w_nat, st)
                      : (g.F > 32 ? smallk_lds_ks<2, EPI>(g, x, w, y, e, w_nat, st)
                                  : smallk_lds_ks<1, EPI>(g, x, w, y, e, w_nat, st));
    if (rc != ACH_EUNSUPPORTED || w_nat) return rc;
    if (g.KS == 3) {
        if (g.F > 64) return smallk_launch<4, 3, EPI>(g, x, w, y, e, st);
        if (g.F > 32) return smallk_launch<2, 3, EPI>(g, x, w, y, e, st);
        return smallk_launch<1, 3, EPI>(g, x, w, y, e, st);
    }
    if (g.F > 64) return smallk_launch<4, 0, EPI>(g, x, w, y, e, st);
    if (g.F > 32) return smallk_launch<2, 0, EPI>(g, x, w, y, e, st);
    return smallk_launch<1, 0, EPI>(g, x, w, y, e, st);
}

// kg_ok: the call may run both K slices of a tile in one workgroup (forward
// passes; input gradients keep the separate reduction, below)
static FwdPlan fwd_plan(const ConvGeom &g, bool kg_ok = true)
{
    FwdPlan pl;
    const int M = g.F, N = g.B * g.OH * g.OW;
    int K = g.C * g.KS * g.KS;
    // 128-row tiles for every larger filter count: with 4 workgroups per CU
    // the 16x16 layers of darknet run unsplit (512 tiles, no partial sums),
    // measured 1.2% faster on the step than 256 x 128 tiles split in two
    pl.bm = M <= 32 ? 32 : (M <= 64 ? 64 : 128);
    pl.bk = g.KS == 3 ? BIm2col3::BK : (fc_geom(g) && pl.bm == 128 ? FC_BK : 16);
    if (fwd_padded_taps(g)) {  // 5x5: one channel + a zero row per k-tile
        pl.bk = BIm2colK<5>::BK;
        K = g.C * pl.bk;
        if (M > 64 && M <= 96) pl.bm = 96;  // three 32-row MFMA tiles per wave
    } else if (fwd_row_taps(g)) {  // 11x11: two filter rows per k-tile
        pl.bk = BIm2colRow<ROW_KS>::BK;
        K = fwd_row_k(g);
        if (M > 64 && M <= 96) pl.bm = 96;
    } else if (M > 64 && M <= 96 && (M & 3) == 0 && g.KS != 3 && g.KS != 1) {
        pl.bm = 96;  // generic loader, 65-96 filters (AlexNet conv1: 96 of 128 rows)
    }
    const int tiles = ((M + pl.bm - 1) / pl.bm) * ((N + 127) / 128);
    const int ktiles = (K + pl.bk - 1) / pl.bk;
    // k-tiles per slice at least: 8, or 4 of the fully connected GEMMs'
    // 32-wide ones (128 K either way)
    const int min_kt = pl.bk == FC_BK && fc_geom(g) ? 4 : 8;
    int s = 1;
    // the padded-tap kernel fits two workgroups per CU: aim at two rounds
    // (measured 0.5% faster on AlexNet than one).  Input gradients (kg_ok
    // false) whose grid gives one to two workgroups per CU (257-511 tiles:
    // AlexNet's 13x13 layers, 338 and 507 tiles) aim there too, since they
    // share the CUs with the weight-gradient GEMMs (AlexNet step 7.78 ->
    // 7.73 ms, three A/B pairs); a 1024 target for every input gradient
    // (or 768) made darknet's 128- and 256-tile ones 1.2-1.4% slower on the
    // step, and 256 or 128 made them 6.5% slower.
    const bool mid_dgrad = !kg_ok && tiles > 256 && tiles < 512;
    const int target = (fwd_padded_taps(g) || mid_dgrad) ? 1024 : 512;
    if (tiles < target) {
        // rounded, not raised: a grid just short of the target (AlexNet's
        // 13x13 forwards with 384 filters, 507 tiles) runs unsplit rather
        // than paying a reduction pass for a 2x grid (measured 2.4% on
        // AlexNet when its input gradients ran the same rule)
        s = (target + tiles / 2) / tiles;
        if (s > 32) s = 32;
        if (s > ktiles / min_kt) s = ktiles / min_kt;
        if (s < 1) s = 1;
    }
    // Two K groups per 512-thread workgroup (k_mfma_gemm<P, 2>) for 3x3
    // forward passes whose grid gives one or two such workgroups per CU on
    // 256 CUs (filter counts divisible by 4: the two float4-filter loaders of
    // fwd_bm):
    //  - 256 tiles split in two (the 8x8 layers of darknet): both slices of
    //    a tile in one workgroup, added in LDS -- the same sums, without the
    //    partials' HBM round trip and the reduction pass;
    //  - 512 tiles not split (the 16x16 layers): K is halved between the two
    //    groups, doubling the waves per SIMD at the same 64 x 64 wave tile
    //    (256->256@16 forward 134 -> 137 TF/s; the sums become two halves
    //    added, a different but fixed order).
    // Grids in between balance worse than twice as many 256-thread
    // workgroups (AlexNet's 338-tile conv5 forward: step 7.81 -> 7.91 ms).
    // Input gradients (kg_ok false) run beside the weight-gradient GEMMs of
    // the second stream, where 8-wave workgroups find fewer free slots:
    // measured on the darknet step, 6.855 ms without, 6.827 with forward
    // passes only, 6.961 with input gradients only.
    // The two groups share the loop's barriers, so they must run the same
    // number of k-tiles: with an odd k-tile count the shorter slice's group
    // would run one tile past its end, where the 3x3 loaders re-read its last
    // tile.  Such shapes keep one group per workgroup.
    const bool kg_shape = kg_ok && pl.bm == 128 && g.KS == 3 && (g.F & 3) == 0 && !fc_geom(g) &&
                          (ktiles & 1) == 0;
    if (kg_shape && s == 1 && tiles == 512 && ktiles >= 16) s = 2;
    // Fully connected GEMMs (N = the batch: few tiles, K split many ways)
    // run pairs of whole slices in one 512-thread workgroup when that still
    // gives at least 256 workgroups, halving the partial sums; an odd split
    // count is raised by one for it.  Alone: FC7 (4096 -> 4096, batch 128)
    // forward 66.5 -> 56.4 us, input gradient 61.1 -> 51.9 us.
    const bool fc_pairs = fc_geom(g) && pl.bm == 128 && (K % pl.bk) == 0;
    if (fc_pairs && (s & 1) && s > 1 && s + 1 <= ktiles / min_kt && ktiles % (s + 1) == 0) s += 1;
    pl.kchunk = ((ktiles + s - 1) / s) * pl.bk;
    pl.splits = (K + pl.kchunk - 1) / pl.kchunk;
    if (fwd_small_k(g)) pl.splits = 1;  // k_conv_fwd_smallk: whole K per tile
    pl.kg = (kg_shape && pl.splits == 2 && 2 * (pl.kchunk / pl.bk) == ktiles &&
             (tiles <= 256 || tiles == 512)) ? 2 : 1;
    if (fc_pairs && (pl.splits & 1) == 0 && pl.splits * (pl.kchunk / pl.bk) == ktiles &&
        tiles * (pl.splits / 2) >= 256)
        pl.kg = 2;
    return pl;
}

static size_t fwd_part_bytes(const ConvGeom &g, bool kg_ok = true)
{
    const FwdPlan pl = fwd_plan(g, kg_ok);
    if (pl.pslices() <= 1) return 0;
    return (size_t)pl.pslices() * g.F * g.B * g.OH * g.OW * sizeof(float);
}

// EPI: the bias / activation epilogue in the GEMM (used without a K split
// and for tiles of at most 128 rows only)
template <int BM, bool EPI>
static int fwd_bm(const ConvGeom &g, const FwdPlan &pl, const float *x, const float *w,
                  float *y, float *part, const Epi &e, bool w_nat, hipStream_t st)
{
    const int M = g.F, N = g.B * g.OH * g.OW, K = g.C * g.KS * g.KS;
    // pairs of K slices in one workgroup: the problem stores the pairs' sums
    // (finished outputs for two slices)
    const bool kg2 = BM == 128 && pl.kg == 2;
    const int psplits = pl.pslices();
    // the two groups run k-tile counts that must match: every slice whole
    if (kg2 && ((pl.splits & 1) || pl.splits * pl.kchunk != ((K + pl.bk - 1) / pl.bk) * pl.bk))
        return ACH_EINVAL;
    if (g.KS == 3 && (M & 3) == 0 && (g.C & 1) == 0) {
        FwdProblem<BM, BIm2col3F, true, EPI> p{x, w, y, part, g, M, N, K, pl.kchunk, psplits};
        p.e = e;
        if constexpr (BM == 128)
            if (kg2) return launch_gemm<decltype(p), 2>(p, M, N, pl.splits, st);
        return launch_gemm(p, M, N, pl.splits, st);
    }
    if (g.KS == 3 && (M & 3) == 0) {
        FwdProblem<BM, BIm2col3, true, EPI> p{x, w, y, part, g, M, N, K, pl.kchunk, psplits};
        p.e = e;
        if constexpr (BM == 128)
            if (kg2) return launch_gemm<decltype(p), 2>(p, M, N, pl.splits, st);
        return launch_gemm(p, M, N, pl.splits, st);
    }
    if (g.KS == 3) {
        FwdProblem<BM, BIm2col3, false, EPI> p{x, w, y, part, g, M, N, K, pl.kchunk, pl.splits};
        p.e = e;
        return launch_gemm(p, M, N, pl.splits, st);
    }
    if constexpr (BM <= 128) {
        if (fc_geom(g)) {
            const size_t xb = (size_t)N * K * sizeof(float);
            constexpr int FBK = BM == 128 ? FC_BK : 16;
            if (w_nat) {
                FcProblem<BM, false, EPI, true, FBK> p{x, w, y, part, M, N, K, pl.kchunk,
                                                       psplits, xb};
                p.e = e;
                if constexpr (BM == 128)
                    if (kg2) return launch_gemm<decltype(p), 2>(p, M, N, pl.splits, st);
                return launch_gemm(p, M, N, pl.splits, st);
            }
            if ((M & 3) == 0) {
                FcProblem<BM, true, EPI, false, FBK> p{x, w, y, part, M, N, K, pl.kchunk,
                                                       psplits, xb};
                p.e = e;
                if constexpr (BM == 128)
                    if (kg2) return launch_gemm<decltype(p), 2>(p, M, N, pl.splits, st);
                return launch_gemm(p, M, N, pl.splits, st);
            }
            FcProblem<BM, false, EPI, false, FBK> p{x, w, y, part, M, N, K, pl.kchunk, psplits,
                                                    xb};
            p.e = e;
            if constexpr (BM == 128)
                if (kg2) return launch_gemm<decltype(p), 2>(p, M, N, pl.splits, st);
            return launch_gemm(p, M, N, pl.splits, st);
        }
    }
    if (g.KS == 1) {
        FwdProblem<BM, BIm2colAny<1>, false, EPI> p{x, w, y, part, g, M, N, K, pl.kchunk,
                                                     pl.splits};
        p.e = e;
        return launch_gemm(p, M, N, pl.splits, st);
    }
    if constexpr (BM <= 128) {
        if (fwd_padded_taps(g)) {
            FwdProblem<BM, BIm2colK<5>, true, EPI> p{x, w, y, part, g, M, N,
                                                     g.C * BIm2colK<5>::BK, pl.kchunk,
                                                     pl.splits};
            p.e = e;
            return launch_gemm(p, M, N, pl.splits, st);
        }
        if (fwd_row_taps(g)) {
            FwdProblem<BM, BIm2colRow<ROW_KS>, true, EPI> p{x, w, y, part, g, M, N,
                                                             fwd_row_k(g), pl.kchunk, pl.splits};
            p.e = e;
            return launch_gemm(p, M, N, pl.splits, st);
        }
    }
    FwdProblem<BM, BIm2colAny<0>, false, EPI> p{x, w, y, part, g, M, N, K, pl.kchunk, pl.splits};
    p.e = e;
    return launch_gemm(p, M, N, pl.splits, st);
}

// 96-row tiles (one wave column of three 32-row MFMA tiles) for 65-96
// filters with float4 k-major weights: the padded-tap 5x5 path and the
// generic im2col loader (AlexNet's 11x11 first layer); the other loaders
// assume BM | 256 or BM % 64 == 0
template <int BM, bool EPI>
static int fwd_bm_padded(const ConvGeom &g, const FwdPlan &pl, const float *x, const float *w,
                         float *y, float *part, const Epi &e, hipStream_t st)
{
    const int M = g.F, N = g.B * g.OH * g.OW;
    if (fwd_row_taps(g)) {
        FwdProblem<BM, BIm2colRow<ROW_KS>, true, EPI> p{x, w, y, part, g, M, N, fwd_row_k(g),
                                                         pl.kchunk, pl.splits};
        p.e = e;
        return launch_gemm(p, M, N, pl.splits, st);
    }
    if (!fwd_padded_taps(g)) {
        FwdProblem<BM, BIm2colAny<0>, true, EPI> p{x, w, y, part, g, M, N, g.C * g.KS * g.KS,
                                                   pl.kchunk, pl.splits};
        p.e = e;
        return launch_gemm(p, M, N, pl.splits, st);
    }
    FwdProblem<BM, BIm2colK<5>, true, EPI> p{x, w, y, part, g, M, N, g.C * BIm2colK<5>::BK,
                                             pl.kchunk, pl.splits};
    p.e = e;
    return launch_gemm(p, M, N, pl.splits, st);
}

// w: k-major filter Wt[K][M]; part: fwd_part_bytes(g) of scratch (or NULL
// when no split is planned).  An active epilogue e runs in the GEMM when K
// is not split, or in the split-K reduction.
// w_nat: a fully connected geometry's w is the filter itself (W[F][K]).
static int fwd_impl(const ConvGeom &g, const float *x, const float *w, float *y, float *part,
                    hipStream_t st, const Epi &e = Epi(), bool w_nat = false, bool kg_ok = true)
{
    if (fwd_small_k(g))
        return e.active() ? fwd_small_k_launch<true>(g, x, w, y, e, w_nat, st)
                          : fwd_small_k_launch<false>(g, x, w, y, e, w_nat, st);
    const FwdPlan pl = fwd_plan(g, kg_ok);
    const bool unsplit = pl.pslices() == 1;  // no partial sums
    const int ps = pl.pslices();
    const bool gemm_epi = e.active() && unsplit;
    int rc;
    if (gemm_epi) {
        if (pl.bm == 32) rc = fwd_bm<32, true>(g, pl, x, w, y, part, e, w_nat, st);
        else if (pl.bm == 96) rc = fwd_bm_padded<96, true>(g, pl, x, w, y, part, e, st);
        else if (pl.bm == 64) rc = fwd_bm<64, true>(g, pl, x, w, y, part, e, w_nat, st);
        else rc = fwd_bm<128, true>(g, pl, x, w, y, part, e, w_nat, st);
        return rc;
    }
    if (pl.bm == 32) rc = fwd_bm<32, false>(g, pl, x, w, y, part, e, w_nat, st);
    else if (pl.bm == 96) rc = fwd_bm_padded<96, false>(g, pl, x, w, y, part, e, st);
    else if (pl.bm == 64) rc = fwd_bm<64, false>(g, pl, x, w, y, part, e, w_nat, st);
    else rc = fwd_bm<128, false>(g, pl, x, w, y, part, e, w_nat, st);
    if (rc || unsplit) return rc;
    const int M = g.F, N = g.B * g.OH * g.OW;
    const size_t mn = (size_t)M * N;
    const bool al16 = ((reinterpret_cast<uintptr_t>(part) | reinterpret_cast<uintptr_t>(y)) & 15) == 0;
    const FastDiv dM = make_fastdiv((unsigned)M);
    if (fc_geom(g)) {  // FcProblem partials: [z][b][m]
        const bool v4 = al16 && (mn & 3) == 0;
        const dim3 grid(grid_for(v4 ? mn / 4 : mn, 256, 1u << 20));
        if (e.active() && v4)
            hipLaunchKernelGGL((k_splitk_rows<true, true>), grid, dim3(256), 0, st, part, y,
                               (int)mn, dM, ps, e);
        else if (e.active())
            hipLaunchKernelGGL((k_splitk_rows<true, false>), grid, dim3(256), 0, st, part, y,
                               (int)mn, dM, ps, e);
        else if (v4)
            hipLaunchKernelGGL((k_splitk_rows<false, true>), grid, dim3(256), 0, st, part, y,
                               (int)mn, dM, ps, e);
        else
            hipLaunchKernelGGL((k_splitk_rows<false, false>), grid, dim3(256), 0, st, part, y,
                               (int)mn, dM, ps, e);
        return check_launch();
    }
    const int ohw = g.OH * g.OW;
    const FastDiv dohw = make_fastdiv((unsigned)ohw);
    const bool v4 = al16 && (ohw & 3) == 0;  // four positions never straddle a plane
    const dim3 grid(grid_for(v4 ? mn / 4 : mn, 256, 1u << 20));
    if (!v4 && al16 && (N & 3) == 0) {  // float4 loads in the partials' order
        const dim3 g4(grid_for(mn / 4, 256, 1u << 20));
        const FastDiv dN = make_fastdiv((unsigned)N);
        if (e.active())
            hipLaunchKernelGGL((k_splitk_to_nchw_pv<true>), g4, dim3(256), 0, st, part, y, M, N,
                               dohw, dN, ps, e);
        else
            hipLaunchKernelGGL((k_splitk_to_nchw_pv<false>), g4, dim3(256), 0, st, part, y, M, N,
                               dohw, dN, ps, e);
        return check_launch();
    }
    if (e.active() && v4)
        hipLaunchKernelGGL((k_splitk_to_nchw<true, true>), grid, dim3(256), 0, st, part, y, M, N,
                           dohw, dM, ps, e);
    else if (e.active())
        hipLaunchKernelGGL((k_splitk_to_nchw<true, false>), grid, dim3(256), 0, st, part, y, M, N,
                           dohw, dM, ps, e);
    else if (v4)
        hipLaunchKernelGGL((k_splitk_to_nchw<false, true>), grid, dim3(256), 0, st, part, y, M, N,
                           dohw, dM, ps, e);
    else
        hipLaunchKernelGGL((k_splitk_to_nchw<false, false>), grid, dim3(256), 0, st, part, y, M,
                           N, dohw, dM, ps, e);
    return check_launch();
}

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// The chunked K order of the weight gradient applies when padding the
// output plane to whole 16-position chunks wastes at most WGRAD_PAD_WASTE of
// the work; otherwise the (image, position) order splits K to aim at
// ~WGRAD_TARGET workgroups, K chunks a multiple of the k-tile.
constexpr double WGRAD_PAD_WASTE = 0.0625;
static int wgrad_nchunks(const ConvGeom &g) { return (g.OH * g.OW + 15) / 16; }
static bool wgrad_chunked(const ConvGeom &g)
{
    const int ohw = g.OH * g.OW;
    return wgrad_nchunks(g) * 16 - ohw <= WGRAD_PAD_WASTE * ohw;
}

// Cost model of the weight-gradient GEMM plus its split-K reduction, in CU
// cycles.  All workgroups do equal work, so the GEMM takes about
// ceil(workgroups / 256 CUs) times one workgroup's time: its MFMAs (a
// 16-position chunk of `images` images, bm*bn*16 MACs per image at 128 fp32
// MACs per CU cycle) and its epilogue, which writes bm*bn partial sums at a
// CU's share of HBM bandwidth (~15 bytes per cycle); below two workgroups
// per CU the matrix pipes idle (x1.25).  The reduction then reads every
// partial once (~2300 bytes per cycle for the whole chip).  Without the
// epilogue and reduction terms the model asks for tens of thousands of
// workgroups of a few images each on small planes (AlexNet's 13x13 layers).
static double wgrad_cost(long long wgs, int bm, int bn, int images)
{
    const double tile = (double)bm * bn;
    const double per_wg = tile * (images * 16.0 / 128.0 + 4.0 / 15.0);
    double c = (double)((wgs + 255) / 256) * per_wg;
    if (wgs < 512) c *= 1.25;
    return c + (double)wgs * tile * 4.0 / 2300.0;
}

// chunked split: spc splits per position chunk, nbs images each (>= 4 per
// split), the count with the lowest modelled cost (ties: fewer workgroups,
// so fewer partial sums)
static double wgrad_split_chunked(const ConvGeom &g, int bm, int bn, int &splits, int &spc,
                                  int &nbs)
{
    const int M = g.F, N = g.C * g.KS * g.KS, nchunks = wgrad_nchunks(g);
    const long long tiles = (long long)((M + bm - 1) / bm) * ((N + bn - 1) / bn);
    const int max_spc = g.B >= 4 ? g.B / 4 : 1;
    double best = -1;
    for (int want = 1; want <= max_spc && want <= 64; ++want) {
        const int b = (g.B + want - 1) / want, s = (g.B + b - 1) / b;
        const long long wgs = tiles * nchunks * s;
        if (wgs > 65535LL * 1024) break;
        const double c = wgrad_cost(wgs, bm, bn, b);
        if (best < 0 || c < best * (1 - 1e-9)) {
            best = c;
            nbs = b;
            spc = s;
        }
    }
    splits = nchunks * spc;
    return best;
}

static void wgrad_split(const ConvGeom &g, int bm, int bn, int &splits, int &kchunk)
{
    if (wgrad_chunked(g)) {
        int spc, nbs;
        wgrad_split_chunked(g, bm, bn, splits, spc, nbs);
        kchunk = 0;
        return;
    }
    const int M = g.F, N = g.C * g.KS * g.KS, K = g.B * g.OH * g.OW;
    const int tiles = ((M + bm - 1) / bm) * ((N + bn - 1) / bn);
    const int bk = WGRAD_BK;
    int s = (WGRAD_TARGET + tiles - 1) / tiles;
    const int max_s = (K + 4 * bk - 1) / (4 * bk);  // >= 4 k-tiles per split
    if (s > max_s) s = max_s;
    if (s < 1) s = 1;
    if (s > 1024) s = 1024;
    int chunk = (K + s - 1) / s;
    chunk = (chunk + bk - 1) / bk * bk;
    splits = (K + chunk - 1) / chunk;
    kchunk = chunk;
}

// wgrad tile: 32-column tiles when C*k*k <= 32 (e.g. the 3-channel first
// layer, N = 27), otherwise BM from the filter count x 128.
// 65-96 filters (AlexNet's 11x11 first layer): 96 x 128 tiles, each wave
// 96 x 32, instead of a 128-row tile a quarter empty
static bool wgrad_96(const ConvGeom &g)
{
    return g.F > 64 && g.F <= 96 && !fc_geom(g) && g.C * g.KS * g.KS > 32;
}
static int wgrad_bm(const ConvGeom &g)
{
    if (g.C * g.KS * g.KS <= 32 && g.F > 64) return 128;
    if (wgrad_96(g)) return 96;
    return g.F <= 32 ? 32 : (g.F <= 64 ? 64 : 128);
}
// Layers with more than 96 filters in the chunked order take the N tile of
// 64, 96 or 128 columns with the lowest grid cost (ties: fewer workgroups);
// e.g. every config-1 3x3 layer at batch 128 has 1152 (tile, chunk) pairs
// of 128 x 64, which leave a 12%-full second round on 1024 workgroup slots,
// against exactly 3 x 256 workgroups of 128 x 96.
static int wgrad_bn(const ConvGeom &g)
{
    if (fc_geom(g)) return 128;
    if (g.C * g.KS * g.KS <= 32 && g.F > 64) return 32;
    if (wgrad_96(g)) return 128;
    if (g.F <= 64) return 128;
    if (!wgrad_chunked(g)) return 64;
    int best_bn = 64;
    double best = -1;
    long long best_wgs = 0;
    for (int bn : {64, 96, 128}) {
        int splits, spc, nbs;
        const double c = wgrad_split_chunked(g, 128, bn, splits, spc, nbs);
        const long long wgs = (long long)((g.F + 127) / 128) *
                              ((g.C * g.KS * g.KS + bn - 1) / bn) * splits;
        if (best < 0 || c < best * (1 - 1e-9) || (c <= best * (1 + 1e-9) && wgs < best_wgs)) {
            best = c;
            best_bn = bn;
            best_wgs = wgs;
        }
    }
    return best_bn;
}

// sgd: the weights' update for the unsplit chunked and fully connected
// problems (their epilogue applies it); *sgd_done tells the caller
template <int BM, int BN>
static int wgrad_launch(const ConvGeom &g, const float *x, const float *dy, float *dw,
                        float *part, int splits, int kchunk, hipStream_t st, const Sgd &sgd,
                        bool &sgd_done)
{
    const int M = g.F, N = g.C * g.KS * g.KS, K = g.B * g.OH * g.OW;
    WgradDivs dv;
    dv.ohw = make_fastdiv((unsigned)(g.OH * g.OW));
    dv.ow = make_fastdiv((unsigned)g.OW);
    dv.batch = make_fastdiv((unsigned)g.B);
    if (wgrad_chunked(g)) {
        int spc, nbs;
        wgrad_split_chunked(g, BM, BN, splits, spc, nbs);
        if (splits > 65535) return ACH_EUNSUPPORTED;
        const Sgd s1 = splits == 1 ? sgd : Sgd();
        sgd_done = s1.w != nullptr;
        if (g.KS == 3) {
            WgradProblemC<BM, BN, 3> p{x, dy, dw, part, g, dv, M, N, spc, nbs, splits, s1};
            return launch_gemm(p, M, N, splits, st);
        }
        if (g.KS == 1) {
            WgradProblemC<BM, BN, 1> p{x, dy, dw, part, g, dv, M, N, spc, nbs, splits, s1};
            return launch_gemm(p, M, N, splits, st);
        }
        WgradProblemC<BM, BN, 0> p{x, dy, dw, part, g, dv, M, N, spc, nbs, splits, s1};
        return launch_gemm(p, M, N, splits, st);
    }
    if (g.KS == 3) {
        WgradProblem<BM, BN, 3> p{x, dy, dw, part, g, dv, M, N, K, kchunk, splits};
        return launch_gemm(p, M, N, splits, st);
    }
    if (g.KS == 1) {
        WgradProblem<BM, BN, 1> p{x, dy, dw, part, g, dv, M, N, K, kchunk, splits};
        return launch_gemm(p, M, N, splits, st);
    }
    WgradProblem<BM, BN, 0> p{x, dy, dw, part, g, dv, M, N, K, kchunk, splits};
    return launch_gemm(p, M, N, splits, st);
}

template <int BM>
static int fc_wgrad_bm(const ConvGeom &g, const float *x, const float *dy, float *dw,
                       float *part, int splits, int kchunk, hipStream_t st, const Sgd &sgd)
{
    const int M = g.F, N = g.C, K = g.B;
    const size_t xb = (size_t)K * N * sizeof(float);
    if ((M & 3) == 0) {
        FcWgradProblem<BM, true> p{x, dy, dw, part, M, N, K, kchunk, splits, xb, sgd};
        return launch_gemm(p, M, N, splits, st);
    }
    FcWgradProblem<BM, false> p{x, dy, dw, part, M, N, K, kchunk, splits, xb, sgd};
    return launch_gemm(p, M, N, splits, st);
}

static int fc_wgrad_launch(const ConvGeom &g, const float *x, const float *dy, float *dw,
                           float *part, int bm, int splits, int kchunk, hipStream_t st,
                           const Sgd &sgd, bool &sgd_done)
{
    const Sgd s1 = splits == 1 ? sgd : Sgd();
    sgd_done = s1.w != nullptr;
    if (bm == 32) return fc_wgrad_bm<32>(g, x, dy, dw, part, splits, kchunk, st, s1);
    if (bm == 64) return fc_wgrad_bm<64>(g, x, dy, dw, part, splits, kchunk, st, s1);
    return fc_wgrad_bm<128>(g, x, dy, dw, part, splits, kchunk, st, s1);
}

// the one-pass weight gradient of 1x1 stride-1 layers (not fully connected)
// with at most 16 filters on planes of at most 256 positions, a multiple of
// 4 (a classifier's last layer): every workgroup reads dy (F/2 times the
// bytes of x in all, from L2), x is read once
constexpr int WG1_FMAX = 16, WG1_CB = 2;
static bool wgrad_1x1_smallf(const ConvGeom &g)
{
    return g.KS == 1 && g.S == 1 && g.P == 0 && !fc_geom(g) && g.F <= WG1_FMAX &&
           g.OH * g.OW <= 256 && (g.OH * g.OW) % 4 == 0;
}
static int wgrad_1x1_smallf_launch(const ConvGeom &g, const float *x, const float *dy, float *dw,
                                   const Sgd &sg, hipStream_t st)
{
    hipLaunchKernelGGL((k_wgrad_1x1_smallf<WG1_FMAX, WG1_CB>), dim3((g.C + WG1_CB - 1) / WG1_CB),
                       dim3(WG1_NT), 0, st, x, dy, dw, g.B, g.C, g.F, g.OH * g.OW, sg);
    return check_launch();
}

// the small-channel input gradient: stride 1, at most 4 input channels,
// kernels up to 16 wide, a staged chunk that fits LDS
static size_t dgrad_small_c_lds(const ConvGeom &g, int nc)
{
    const int PH = DG_TH + g.KS - 1, PWd = (DG_TW + g.KS - 1 + 3) & ~3, FC = dg_fc(g.KS);
    const size_t stage = (size_t)FC * PH * PWd + 4 * FC * g.KS * g.KS;
    const size_t red = (size_t)(DG_WAVES - 1) * nc * 4 * 64;
    return (stage > red ? stage : red) * sizeof(float);
}
static bool dgrad_small_c(const ConvGeom &g)
{
    // the chunk's patch rows fit the per-wave register prefetch
    const int PH = DG_TH + g.KS - 1;
    // (and one image's dy addressable by 32-bit buffer offsets)
    return g.S == 1 && g.P <= g.KS - 1 && g.C <= 4 && g.KS <= 16 &&
           (dg_fc(g.KS) / DG_WAVES) * PH <= dg_rows(g.KS) * 4 &&
           dgrad_small_c_lds(g, 4) <= 65536 && (long long)g.F * g.OH * g.OW * 4 < (1ll << 31);
}

template <int NC>
static int dgrad_small_c_nc(const ConvGeom &g, const float *dy, const float *w, float *dx,
                            hipStream_t st)
{
    const size_t lds = dgrad_small_c_lds(g, NC);
    const int tiles_x = (g.W + DG_TW - 1) / DG_TW, tiles_y = (g.H + DG_TH - 1) / DG_TH;
    const dim3 grid(tiles_x * tiles_y, g.B);
    if (grid.y > 65535) return ACH_EUNSUPPORTED;
    if (g.KS == 3)
        hipLaunchKernelGGL((k_conv_dgrad_smallc<NC, 3>), grid, dim3(DG_NT), lds, st, dy, w, dx, g,
                           tiles_x);
    else if (g.KS == 5)
        hipLaunchKernelGGL((k_conv_dgrad_smallc<NC, 5>), grid, dim3(DG_NT), lds, st, dy, w, dx, g,
                           tiles_x);
    else
        hipLaunchKernelGGL((k_conv_dgrad_smallc<NC, 0>), grid, dim3(DG_NT), lds, st, dy, w, dx, g,
                           tiles_x);
    return check_launch();
}

static int dgrad_small_c_launch(const ConvGeom &g, const float *dy, const float *w, float *dx,
                                hipStream_t st)
{
    switch (g.C) {
    case 1: return dgrad_small_c_nc<1>(g, dy, w, dx, st);
    case 2: return dgrad_small_c_nc<2>(g, dy, w, dx, st);
    case 3: return dgrad_small_c_nc<3>(g, dy, w, dx, st);
    default: return dgrad_small_c_nc<4>(g, dy, w, dx, st);
    }
}

}  // namespace ach

using namespace ach;

extern "C" {

int ach_conv_out_h(const ach_conv_desc *d) { return conv_ok(d) ? geom(d).OH : -1; }
int ach_conv_out_w(const ach_conv_desc *d) { return conv_ok(d) ? geom(d).OW : -1; }

// Workspace of the forward pass: the k-major copy of the filter, then the
// split-K partials when the plan splits K.
size_t ach_conv_fwd_workspace(const ach_conv_desc *d)
{
    if (!conv_ok(d)) return 0;
    const ConvGeom g = geom(d);
    if (conv_xy(d)) return xy_col_bytes(g);
    return align256((size_t)g.F * g.C * g.KS * g.KS * sizeof(float)) + fwd_part_bytes(g);
}

int ach_conv_fwd(const ach_conv_desc *d, const float *x, const float *w, float *y,
                 void *ws, size_t ws_bytes, ach_stream_t stream)
{
    if (!conv_ok(d) || !x || !w || !y) return ACH_EINVAL;
    if (!fits_int(d)) return ACH_EUNSUPPORTED;
    if (!ws || ws_bytes < ach_conv_fwd_workspace(d)) return ACH_EWORKSPACE;
    if (conv_xy(d)) return xy_fwd(d, x, w, false, y, ws, ws_bytes, stream);
    const ConvGeom g = geom(d);
    hipStream_t st = as_stream(stream);
    const int M = g.F, K = g.C * g.KS * g.KS;
    float *wt = (float *)ws;
    float *part = (float *)((char *)ws + align256((size_t)M * K * sizeof(float)));
    // a fully connected geometry reads the filter in its own layout, and so
    // does the patch-staged shallow-im2col kernel
    if (fc_geom(g)) return fwd_impl(g, x, w, y, part, st, Epi(), true);
    if (fwd_small_k(g)) {
        const int rc0 = fwd_small_k_launch<false>(g, x, w, y, Epi(), true, st);
        if (rc0 != ACH_EUNSUPPORTED) return rc0;
    }
    hipLaunchKernelGGL(k_weights_kmajor, dim3((K + 31) / 32, (M + 31) / 32), dim3(256), 0, st, w,
                       wt, M, K);
    int rc = check_launch();
    if (rc) return rc;
    return fwd_impl(g, x, wt, y, part, st);
}

// geometry of stride-1 dgrad seen as a forward convolution of dy
static ConvGeom dgrad_as_fwd(const ConvGeom &g)
{
    ConvGeom t;
    t.B = g.B; t.C = g.F; t.H = g.OH; t.W = g.OW;
    t.F = g.C; t.KS = g.KS; t.S = 1; t.P = g.KS - 1 - g.P;
    t.OH = g.H; t.OW = g.W;
    t.dkk = g.dkk; t.dks = g.dks;
    return t;
}

size_t ach_conv_bwd_data_workspace(const ach_conv_desc *d)
{
    if (!conv_ok(d)) return 0;
    const ConvGeom g = geom(d);
    if (conv_xy(d)) return xy_col_bytes(g);
    size_t wf = (size_t)g.F * g.C * g.KS * g.KS * sizeof(float);
    if (g.S == 1 && g.P <= g.KS - 1) return align256(wf) + fwd_part_bytes(dgrad_as_fwd(g), false);
    // strided fallback: one image's column buffer
    return (size_t)g.C * g.KS * g.KS * g.OH * g.OW * sizeof(float);
}

int ach_conv_bwd_data(const ach_conv_desc *d, const float *dy, const float *w, float *dx,
                      void *ws, size_t ws_bytes, ach_stream_t stream)
{
    if (!conv_ok(d) || !dy || !w || !dx) return ACH_EINVAL;
    if (!fits_int(d)) return ACH_EUNSUPPORTED;
    const size_t need = ach_conv_bwd_data_workspace(d);
    if (!ws || ws_bytes < need) return ACH_EWORKSPACE;
    const ConvGeom g = geom(d);
    hipStream_t st = as_stream(stream);
    const bool xy = conv_xy(d);
    if (!xy && dgrad_small_c(g) && !fc_geom(g)) return dgrad_small_c_launch(g, dy, w, dx, st);
    if (!xy && g.S == 1 && g.P <= g.KS - 1) {
        const size_t tot = (size_t)g.F * g.C * g.KS * g.KS;
        float *part = (float *)((char *)ws + align256(tot * sizeof(float)));
        // 1x1: the flipped k-major filter Wft[f][c] is W itself
        if (g.KS == 1) return fwd_impl(dgrad_as_fwd(g), dy, w, dx, part, st, Epi(), false, false);
        float *wf = (float *)ws;
        hipLaunchKernelGGL(k_weights_flip_kmajor, dim3(grid_for(tot, 256)), dim3(256), 0, st, w,
                           wf, g.F, g.C, g.KS * g.KS);
        int rc = check_launch();
        if (rc) return rc;
        return fwd_impl(dgrad_as_fwd(g), dy, wf, dx, part, st, Epi(), false, false);
    }
    // Strided convolution (unequal strides included): the reference's
    // per-image TN GEMM + col2im (ConvolutionalLayer.c:933-945).  Not on any
    // benchmark path.
    const int m = g.F, n = g.C * g.KS * g.KS, k = g.OH * g.OW;
    float *col = (float *)ws;
    for (int i = 0; i < g.B; ++i) {
        int rc = ach_gemm(1, 0, n, k, m, 1.f, w, n, dy + (size_t)i * m * k, k, 0.f, col, k,
                          stream);
        if (rc) return rc;
        rc = ach_col2im(col, g.C, g.H, g.W, g.KS, g.KS, g.P, g.P, stride_h(d), d->stride, 1, 1,
                        dx + (size_t)i * g.C * g.H * g.W, stream);
        if (rc) return rc;
    }
    return ACH_OK;
}

// ---- prepared filters ----------------------------------------------------
static bool dgrad_flips(const ConvGeom &g) { return g.S == 1 && g.P <= g.KS - 1 && g.KS > 1; }

int ach_conv_prepare_filters(int njobs, const ach_filter_job *jobs, ach_stream_t stream)
{
    if (njobs < 0 || (njobs > 0 && !jobs)) return ACH_EINVAL;
    hipStream_t st = as_stream(stream);
    for (int j0 = 0; j0 < njobs; j0 += PREP_MAX_JOBS) {
        PrepTable tab;
        tab.n = 0;
        long long blocks = 0;
        for (int j = j0; j < njobs && j < j0 + PREP_MAX_JOBS; ++j) {
            const ach_filter_job &q = jobs[j];
            if (!conv_ok(&q.desc) || !q.w || !q.wt) return ACH_EINVAL;
            const ConvGeom g = geom(&q.desc);
            PrepJob &J = tab.job[tab.n++];
            J.w = q.w;
            J.wt = q.wt;
            J.wft = q.wft;
            J.M = g.F;
            J.C = g.C;
            J.KK = g.KS * g.KS;
            const int K = J.C * J.KK;
            // fully connected geometry: the forward reads W itself, no copy
            J.tiles_t = fc_geom(g) ? 0 : ((K + 31) / 32) * ((J.M + 31) / 32);
            J.tiles_f = 0;
            if (q.wft && dgrad_flips(g) && !conv_xy(&q.desc))
                J.tiles_f = (int)(((long long)J.M * J.C + 255) / 256);
            blocks += J.tiles_t + J.tiles_f;
        }
        if (blocks > 0x7fffffffLL) return ACH_EUNSUPPORTED;
        if (blocks == 0) continue;
        hipLaunchKernelGGL(k_prepare_filters, dim3((unsigned)blocks), dim3(256), 0, st, tab);
        int rc = check_launch();
        if (rc) return rc;
    }
    return ACH_OK;
}

int ach_conv_fwd_prepared(const ach_conv_desc *d, const float *x, const float *wt, float *y,
                          void *ws, size_t ws_bytes, ach_stream_t stream)
{
    if (!conv_ok(d) || !x || !wt || !y) return ACH_EINVAL;
    if (!fits_int(d)) return ACH_EUNSUPPORTED;
    if (conv_xy(d)) return xy_fwd(d, x, wt, true, y, ws, ws_bytes, stream);
    const ConvGeom g = geom(d);
    const size_t need = fwd_part_bytes(g);
    if (need && (!ws || ws_bytes < need)) return ACH_EWORKSPACE;
    return fwd_impl(g, x, wt, y, (float *)ws, as_stream(stream), Epi(), fc_geom(g));
}

int ach_conv_is_fully_connected(const ach_conv_desc *d)
{
    return conv_ok(d) && fc_geom(geom(d)) ? 1 : 0;
}

int ach_conv_fwd_bias_act_prepared(const ach_conv_desc *d, const float *x, const float *wt,
                                   const float *bias, int activation, float *y, void *ws,
                                   size_t ws_bytes, ach_stream_t stream)
{
    if (!conv_ok(d) || !x || !wt || !y) return ACH_EINVAL;
    if (activation != ACH_LOGISTIC && activation != ACH_RELU && activation != ACH_LINEAR &&
        activation != ACH_LEAKY)
        return ACH_EUNSUPPORTED;
    if (!fits_int(d)) return ACH_EUNSUPPORTED;
    const ConvGeom g = geom(d);
    if (conv_xy(d)) {  // the three passes, as ach_conv_fwd_prepared + bias + activation
        int rc = xy_fwd(d, x, wt, true, y, ws, ws_bytes, stream);
        if (!rc && bias) rc = ach_add_bias(y, bias, g.B, g.F, g.OH * g.OW, stream);
        if (rc) return rc;
        return ach_activate(y, (size_t)g.B * g.F * g.OH * g.OW, activation, stream);
    }
    const size_t need = fwd_part_bytes(g);
    if (need && (!ws || ws_bytes < need)) return ACH_EWORKSPACE;
    Epi e;
    e.bias = bias;
    e.slope = activation == ACH_LEAKY ? 0.1 : (activation == ACH_RELU ? 0.0 : 1.0);
    hipStream_t st = as_stream(stream);
    const int rc = fwd_impl(g, x, wt, y, (float *)ws, st, e, fc_geom(g));
    // logistic, with its double exp, runs after the bias epilogue
    if (rc || activation != ACH_LOGISTIC) return rc;
    return ach_activate(y, (size_t)g.B * g.F * g.OH * g.OW, activation, stream);
}

int ach_conv_bwd_data_prepared(const ach_conv_desc *d, const float *dy, const float *w,
                               const float *wft, float *dx, void *ws, size_t ws_bytes,
                               ach_stream_t stream)
{
    if (!conv_ok(d) || !dy || !w || !dx) return ACH_EINVAL;
    if (!fits_int(d)) return ACH_EUNSUPPORTED;
    const ConvGeom g = geom(d);
    if (conv_xy(d) || !(g.S == 1 && g.P <= g.KS - 1))
        return ACH_EUNSUPPORTED;  // strided: ach_conv_bwd_data
    if (dgrad_small_c(g) && !fc_geom(g)) return dgrad_small_c_launch(g, dy, w, dx, as_stream(stream));
    if (g.KS > 1 && !wft) return ACH_EINVAL;
    const ConvGeom t = dgrad_as_fwd(g);
    const size_t need = fwd_part_bytes(t, false);
    if (need && (!ws || ws_bytes < need)) return ACH_EWORKSPACE;
    return fwd_impl(t, dy, g.KS == 1 ? w : wft, dx, (float *)ws, as_stream(stream), Epi(), false,
                    false);
}

size_t ach_conv_bwd_filter_workspace(const ach_conv_desc *d)
{
    if (!conv_ok(d)) return 0;
    const ConvGeom g = geom(d);
    if (conv_xy(d)) return xy_col_bytes(g);
    // (the one-pass 1x1 kernel needs none, but unaligned operands take the
    // GEMM, so its workspace is reported)
    int splits, kchunk;
    wgrad_split(g, wgrad_bm(g), wgrad_bn(g), splits, kchunk);
    if (splits <= 1) return 0;
    const int groups = splits > 2 * SPLIT_GROUP ? (splits + SPLIT_GROUP - 1) / SPLIT_GROUP : 0;
    return (size_t)(splits + groups) * g.F * g.C * g.KS * g.KS * sizeof(float);
}

// dw += the weight gradient; with sgd.w, then the weights' SGD step on
// (w, dw) in the pass that finishes dw (the GEMM's unsplit epilogue or the
// split-K reduction), else by ach_sgd_update after it
static int bwd_filter(const ach_conv_desc *d, const float *x, const float *dy, float *dw,
                      void *ws, size_t ws_bytes, ach_stream_t stream, const Sgd &sgd)
{
    if (!conv_ok(d) || !x || !dy || !dw) return ACH_EINVAL;
    if (!fits_int(d)) return ACH_EUNSUPPORTED;
    const ConvGeom g = geom(d);
    if (conv_xy(d)) {
        const int rc = xy_bwd_filter(d, x, dy, dw, ws, ws_bytes, stream);
        if (rc || !sgd.w) return rc;
        return ach_sgd_update((size_t)g.F * g.C * g.KS * g.KS, sgd.w, dw, sgd.dc, sgd.lc, sgd.mom,
                              stream);
    }
    // (float4 loads: 16-byte aligned operands; planes are multiples of 4)
    if (wgrad_1x1_smallf(g) &&
        ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(dy)) & 15) == 0)
        return wgrad_1x1_smallf_launch(g, x, dy, dw, sgd, as_stream(stream));
    const int bm = wgrad_bm(g), bn = wgrad_bn(g);
    int splits, kchunk;
    wgrad_split(g, bm, bn, splits, kchunk);
    const size_t need = ach_conv_bwd_filter_workspace(d);
    if (need && (!ws || ws_bytes < need)) return ACH_EWORKSPACE;
    hipStream_t st = as_stream(stream);
    float *part = (float *)ws;
    int rc;
    bool done = false;  // the update was applied in the GEMM's epilogue
    if (fc_geom(g)) rc = fc_wgrad_launch(g, x, dy, dw, part, bm, splits, kchunk, st, sgd, done);
    else if (bn == 32) rc = wgrad_launch<128, 32>(g, x, dy, dw, part, splits, kchunk, st, sgd, done);
    else if (bn == 64) rc = wgrad_launch<128, 64>(g, x, dy, dw, part, splits, kchunk, st, sgd, done);
    else if (bn == 96) rc = wgrad_launch<128, 96>(g, x, dy, dw, part, splits, kchunk, st, sgd, done);
    else if (bm == 96) rc = wgrad_launch<96, 128>(g, x, dy, dw, part, splits, kchunk, st, sgd, done);
    else if (bm == 32) rc = wgrad_launch<32, 128>(g, x, dy, dw, part, splits, kchunk, st, sgd, done);
    else if (bm == 64) rc = wgrad_launch<64, 128>(g, x, dy, dw, part, splits, kchunk, st, sgd, done);
    else rc = wgrad_launch<128, 128>(g, x, dy, dw, part, splits, kchunk, st, sgd, done);
    if (rc) return rc;
    if (splits == 1) {
        if (!sgd.w || done) return ACH_OK;
        return ach_sgd_update((size_t)g.F * g.C * g.KS * g.KS, sgd.w, dw, sgd.dc, sgd.lc, sgd.mom,
                              stream);
    }
    const size_t mn = (size_t)g.F * g.C * g.KS * g.KS;
    // float4 when every slice starts 16-byte aligned (part is a workspace)
    const bool v4 = (mn & 3) == 0 && ((reinterpret_cast<uintptr_t>(part) |
                                       reinterpret_cast<uintptr_t>(dw) |
                                       reinterpret_cast<uintptr_t>(sgd.w)) & 15) == 0;
    const size_t nt = v4 ? mn / 4 : mn;  // threads' outputs
    if (splits > 2 * SPLIT_GROUP) {
        const int groups = (splits + SPLIT_GROUP - 1) / SPLIT_GROUP;
        float *tmp = part + (size_t)splits * mn;
        if (v4)
            hipLaunchKernelGGL(k_splitk_group<true>, dim3(grid_for(nt, 256, 1024), groups),
                               dim3(256), 0, st, part, tmp, mn, splits);
        else
            hipLaunchKernelGGL(k_splitk_group<false>, dim3(grid_for(nt, 256, 1024), groups),
                               dim3(256), 0, st, part, tmp, mn, splits);
        rc = check_launch();
        if (rc) return rc;
        if (v4)
            hipLaunchKernelGGL(k_splitk_reduce<true>, dim3(grid_for(nt, 256)), dim3(256), 0, st,
                               tmp, dw, mn, groups, sgd);
        else
            hipLaunchKernelGGL(k_splitk_reduce<false>, dim3(grid_for(nt, 256)), dim3(256), 0, st,
                               tmp, dw, mn, groups, sgd);
        return check_launch();
    }
    if (v4)
        hipLaunchKernelGGL(k_splitk_reduce<true>, dim3(grid_for(nt, 256)), dim3(256), 0, st, part,
                           dw, mn, splits, sgd);
    else
        hipLaunchKernelGGL(k_splitk_reduce<false>, dim3(grid_for(nt, 256)), dim3(256), 0, st, part,
                           dw, mn, splits, sgd);
    return check_launch();
}

int ach_conv_bwd_filter(const ach_conv_desc *d, const float *x, const float *dy, float *dw,
                        void *ws, size_t ws_bytes, ach_stream_t stream)
{
    return bwd_filter(d, x, dy, dw, ws, ws_bytes, stream, Sgd());
}

int ach_conv_bwd_filter_sgd(const ach_conv_desc *d, const float *x, const float *dy, float *w,
                            float *dw, float decay_coef, float lr_coef, float momentum, void *ws,
                            size_t ws_bytes, ach_stream_t stream)
{
    if (!w) return ACH_EINVAL;
    Sgd sgd;
    sgd.w = w;
    sgd.dc = decay_coef;
    sgd.lc = lr_coef;
    sgd.mom = momentum;
    return bwd_filter(d, x, dy, dw, ws, ws_bytes, stream, sgd);
}

int ach_conv_bwd_data_reads_w(const ach_conv_desc *d)
{
    if (!conv_ok(d) || conv_xy(d)) return 1;
    const ConvGeom g = geom(d);
    // ach_conv_bwd_data_prepared reads wft only for the GEMM path of a
    // stride-1 layer whose filter is wider than 1x1
    return !(g.S == 1 && g.P <= g.KS - 1 && g.KS > 1 && !fc_geom(g) && !dgrad_small_c(g));
}

int ach_gemm(int TA, int TB, int M, int N, int K, float ALPHA, const float *A, int lda,
             const float *B, int ldb, float BETA, float *C, int ldc, ach_stream_t stream)
{
    if (M < 0 || N < 0 || K < 0 || !C) return ACH_EINVAL;
    if (M == 0 || N == 0) return ACH_OK;
    if (K > 0 && (!A || !B)) return ACH_EINVAL;
    const size_t abytes = (size_t)(TA ? K : M) * lda * 4, bbytes = (size_t)(TB ? N : K) * ldb * 4;
    if (abytes >= 0x80000000ull || bbytes >= 0x80000000ull) return ACH_EUNSUPPORTED;
    hipStream_t st = as_stream(stream);
#define ACH_GM(ta, tb)                                                                      \
    {                                                                                       \
        GemmProblem<ta, tb> p{A, B, C, M, N, K, lda, ldb, ldc, abytes, bbytes, ALPHA, BETA}; \
        return launch_gemm(p, M, N, 1, st);                                                 \
    }
    if (!TA && !TB) ACH_GM(false, false)
    if (TA && !TB) ACH_GM(true, false)
    if (!TA && TB) ACH_GM(false, true)
    ACH_GM(true, true)
#undef ACH_GM
}

}  // extern "C"
