#pragma once
// fp32 primitives of the Qwen3.5 forward pass on one MI355X.
//
// Drop-in for the reference's include/forward_pass.h:21-54: the same functions with the same
// signatures and meaning, on host pointers, so engine code written against the reference
// compiles and links against libq35.so unchanged. Weights are nn.Linear row-major
// [out_dim][in_dim]: y[o] = sum_i W[o * in_dim + i] * x[i].
//
// The scalar activations are inline, as in the reference. The other functions run the
// library's gfx950 kernels: the inputs are copied into a device staging buffer the library
// makes once (64 MiB, at the first call), the kernel runs, the outputs are copied back
// before the call returns; matmuls larger than the buffer go through it in blocks of rows.
// No device memory is allocated per call. The functions serialise on the staging buffer, so
// threads may call them concurrently. They return nothing, like the reference's: a failure
// of the device (no GPU, a HIP error) is reported on stderr and ends the process, because
// the caller has no way to see it and there is no CPU path to fall back to.
//
// The decode step and the prefill do not use these functions: their kernels fuse the same
// arithmetic into the projections and mixers.
#include <cmath>
#include <cstddef>
#include <cstdint>

#include "weight_view.h"

inline float silu(float x) { return x / (1.0f + expf(-x)); }
inline float sigmoidf(float x) { return 1.0f / (1.0f + expf(-x)); }
// log(1 + e^x), passing x through above 20
inline float softplusf(float x) { return x > 20.0f ? x : std::log1p(std::exp(x)); }

// x /= sqrt(sum(x^2) + eps), in place (a sum, not a mean: the GDN q / k norm).
void l2norm(float* x, int n, float eps);

// y = W x with fp32 weights.
void matmul(const float* W, const float* x, float* y, int out_dim, int in_dim);

// y = W x with the weights read in place from a checkpoint view: bf16 widened exactly to
// fp32, or fp32.
void matmul(const WeightView& W, const float* x, float* y, int out_dim, int in_dim);

// y = x * rsqrt(mean(x^2) + eps) * (1 + weight): the stored weight is a delta from 1.
void rmsnorm(const float* x, const float* weight, float* y, int n, float eps);

// y = weight * (x * rsqrt(mean(x^2) + eps)) * silu(gate): the plain weight (the GDN norm).
void rmsnorm_gated(const float* x, const float* weight, const float* gate, float* y, int n, float eps);

// Partial rotate-half RoPE in place on one head vector: pairs (i, i + rotary_dim / 2) for
// i < rotary_dim / 2 are rotated by pos * theta^(-2i / rotary_dim); dims from rotary_dim on
// are untouched.
void apply_rope(float* vec, int rotary_dim, int pos, double theta);
