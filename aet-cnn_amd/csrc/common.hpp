// Shared helpers for the gfx950 kernels behind include/aetcnn_ops.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "aetcnn_ops.h"

namespace ach {

// Records the last HIP error string for ach_last_hip_error().
void set_hip_error(hipError_t e);
// Records a message of this library for ach_last_hip_error().
void set_error_message(const char *msg);

// Devices whose per-device state (the device address of a file-scope
// scratch array) the library caches.
constexpr int ACH_MAX_DEVICES = 64;

inline int check_launch()
{
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_hip_error(e);
        return ACH_EHIP;
    }
    return ACH_OK;
}

inline int check(hipError_t e)
{
    if (e != hipSuccess) {
        set_hip_error(e);
        return ACH_EHIP;
    }
    return ACH_OK;
}

inline hipStream_t as_stream(ach_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

constexpr int kWave = 64;

// Grid size for an elementwise kernel: enough blocks to fill 256 CUs several
// times over, capped so a grid-stride loop covers the rest.
inline unsigned grid_for(size_t n, int block, unsigned cap = 256u * 16u)
{
    size_t g = (n + block - 1) / block;
    if (g < 1) g = 1;
    if (g > cap) g = cap;
    return (unsigned)g;
}

// Unsigned division by a runtime constant d: q = (mulhi(n, mul) + n) >> shift
// with shift = ceil(log2 d), mul = floor(2^32 (2^shift - d) / d) + 1
// (Granlund & Montgomery 1994), exact for n < 2^31.
struct FastDiv {
    unsigned mul, shift, d;
};

inline FastDiv make_fastdiv(unsigned d)
{
    FastDiv f;
    unsigned l = 0;
    while ((1ull << l) < d) ++l;
    f.mul = (unsigned)((((1ull << 32) * ((1ull << l) - d)) / d) + 1);
    f.shift = l;
    f.d = d;
    return f;
}

__device__ __forceinline__ int fdiv(int n, const FastDiv &f)
{
    return (int)((__umulhi((unsigned)n, f.mul) + (unsigned)n) >> f.shift);
}

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ double wave_sum(double v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// Activations with the reference's arithmetic (Activation.h:53-61,87-104):
// leaky forward multiplies by the double constant .1 and rounds to float.
__device__ __forceinline__ float act_forward(float x, int act)
{
    if (act == ACH_LEAKY) return (x > 0.f) ? x : (float)(0.1 * (double)x);
    if (act == ACH_RELU) return x * (float)(x > 0.f);
    if (act == ACH_LOGISTIC) return (float)(1. / (1. + exp(-(double)x)));
    return x;
}

__device__ __forceinline__ float act_gradient(float y, int act)
{
    if (act == ACH_LEAKY) return (y > 0.f) ? 1.f : 0.1f;
    if (act == ACH_RELU) return (float)(y > 0.f);
    if (act == ACH_LOGISTIC) return (1.f - y) * y;
    return 1.f;
}

// One SGD step of a parameter a and its update accumulator u
// (ConvolutionalLayer.update, ConvolutionalLayer.c:959-980, via WeightData
// addWeightToUpdates / addUpdatesToWeight / scaleUpdates):
// u += dc*a (dc = -decay*batch); a += lc*u (lc = lr/batch); u *= mom.
// Shared by the flat update and the weight-gradient passes that apply it
// where dW is final, so both compile to the same arithmetic.
__device__ __forceinline__ void sgd_step(float &a, float &u, float dc, float lc, float mom)
{
    u += dc * a;
    a += lc * u;
    u *= mom;
}

// The update a weight-gradient pass applies to (w, dW) once dW is final
// (w == nullptr: none).
struct Sgd {
    float *w = nullptr;
    float dc = 0.f, lc = 0.f, mom = 0.f;
};

// Counter-based uniform in [0,1): SplitMix64 finaliser over
// (seed, iteration, layer, index); top 24 bits.
__host__ __device__ __forceinline__ float dropout_uniform(uint64_t seed, uint32_t iter,
                                                          uint32_t layer, uint32_t i)
{
    uint64_t z = seed + 0x9E3779B97F4A7C15ull * ((((uint64_t)layer) << 32) | iter);
    z ^= (uint64_t)i * 0xD1B54A32D192ED03ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return (float)(uint32_t)(z >> 40) * (1.0f / 16777216.0f);
}

}  // namespace ach
