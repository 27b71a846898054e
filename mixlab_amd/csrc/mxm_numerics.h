// Arithmetic contract shared by every kernel of libmixmoe.
//
// Routing must be bit-exact against the CPU restatement of
// gpu/ir.cpp:1106-1111 (softmax, argsort, renorm), so every value that feeds a
// top-k decision is produced by a fixed sequence of IEEE-754 fp32 operations
// that a C compiler on the host reproduces exactly:
//   * the library is compiled with -ffp-contract=off; fused multiply-adds are
//     written as explicit fmaf where intended;
//   * router logits split d into chunks of MXM_LOGIT_CHUNK from d = 0: each
//     chunk's partial is an fmaf chain over its d in ascending order from +0,
//     and the logit is +0 plus the partials added in ascending chunk order
//     (chunks can be computed in parallel; the additions are sequential);
//   * exp is not the device libm's: mxm_exp below is Cody & Waite (1980)
//     argument reduction e^x = 2^n e^r, n = rint(x log2 e), r = x - n ln2
//     with ln2 split into a 17-bit head and a tail (the split published with
//     Cephes' expf), followed by the degree-7 Taylor polynomial of e^r on
//     |r| <= ln2/2 evaluated by Horner's rule with fmaf.  Truncation error is
//     r^8/8! < 6e-9 relative, under one fp32 ulp;
//   * results that would be subnormal are flushed to +0 explicitly, so the
//     device denormal mode never matters;
//   * bf16 is rounded to nearest-even from fp32 bits.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define MXM_HD __host__ __device__ __forceinline__

// d per chunk of the router logits' summation order (see above)
#define MXM_LOGIT_CHUNK 64

MXM_HD uint32_t mxm_f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
MXM_HD float mxm_u2f(uint32_t u) { return __builtin_bit_cast(float, u); }

// bf16 <-> fp32 (bf16 kept as its 16-bit pattern).
MXM_HD float mxm_bf2f(uint16_t h) { return mxm_u2f(((uint32_t)h) << 16); }
MXM_HD uint16_t mxm_f2bf(float f) {
  const uint32_t u = mxm_f2u(f);
  const uint32_t rounded = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  const uint32_t quiet_nan = (u >> 16) | 0x0040u;
  // a select, not a branch: this sits in every epilogue
  return (uint16_t)(((u & 0x7fffffffu) > 0x7f800000u) ? quiet_nan : rounded);
}
// Round an fp32 value to the nearest bf16 and widen it back.
MXM_HD float mxm_rbf(float f) { return mxm_bf2f(mxm_f2bf(f)); }

// Flush fp32 subnormals to +0 (both signs of tiny results become +0).
MXM_HD float mxm_ftz(float f) {
  return ((mxm_f2u(f) & 0x7f800000u) == 0u) ? 0.0f : f;
}

MXM_HD float mxm_exp(float x) {
  // The range cases are selected at the end rather than branched on; inside
  // [-86.5, 88] the operations are exactly those of the polynomial path.
  const float xc = (x > 88.0f) ? 88.0f : ((x < -86.5f || !(x == x)) ? -86.5f : x);
  const float n = __builtin_rintf(xc * 1.4426950408889634f);
  float r = __builtin_fmaf(-n, 0.693145751953125f, xc);
  r = __builtin_fmaf(-n, 1.4286068203094172e-06f, r);
  float p = 1.9841269841269841e-04f;                 // 1/5040
  p = __builtin_fmaf(p, r, 1.3888888888888889e-03f);  // 1/720
  p = __builtin_fmaf(p, r, 8.3333333333333333e-03f);  // 1/120
  p = __builtin_fmaf(p, r, 4.1666666666666667e-02f);  // 1/24
  p = __builtin_fmaf(p, r, 1.6666666666666667e-01f);  // 1/6
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  const uint32_t bits = (uint32_t)((int)n + 127) << 23;
  const float y = p * mxm_u2f(bits);
  return !(x == x) ? x : (x > 88.0f ? __builtin_inff() : (x < -86.5f ? 0.0f : y));
}

MXM_HD float mxm_sigmoid(float x) { return 1.0f / (1.0f + mxm_exp(-x)); }

MXM_HD float mxm_tanh(float x) {
  const float a = __builtin_fabsf(x);
  const float t = mxm_exp(-2.0f * a);
  const float y = (1.0f - t) / (1.0f + t);
  return __builtin_copysignf(y, x);
}

// Tanh-approximate GELU in the operation order of gpu/ir.cpp:1054-1056:
//   0.5*v * (1 + tanh(0.7978845608 * (v + (0.044715*v) * square(v)))).
// `sq` is square(v); the bf16 flow passes it already rounded to bf16 (MLX's
// square keeps the input dtype, the float scalars promote the rest to fp32).
MXM_HD float mxm_gelu_tanh_sq(float v, float sq) {
  const float a = 0.044715f * v;
  const float b = a * sq;
  const float c = v + b;
  const float d = 0.7978845608f * c;
  const float t = mxm_tanh(d);
  const float e = 1.0f + t;
  const float f = 0.5f * v;
  return f * e;
}

// Expert types and activations: arch/moe.go:8-19, gpu/ir.cpp:1040-1051.
enum {
  MXM_EXPERT_SWIGLU = 0,
  MXM_EXPERT_GEGLU = 1,
  MXM_EXPERT_MLP = 2,
};
enum {
  MXM_ACT_SILU = 0,
  MXM_ACT_GELU = 1,
  MXM_ACT_RELU = 2,
  MXM_ACT_LEAKY_RELU_SQ = 3,
};

// Whether the bf16 flow keeps the hidden (and so y) in bf16: MLX promotes
// it to fp32 for geglu, mlp gelu and mlp leaky_relu_sq, whose float scalar
// arrays are fp32 (gpu/ir.cpp:1053-1066, 1133-1145).
MXM_HD bool mxm_hidden_is_bf16(int expert_type, int activation) {
  if (expert_type == 0) return true;   // swiglu
  if (expert_type == 1) return false;  // geglu
  return activation == 0 || activation == 2;  // mlp silu, relu
}

// Hidden activation h = act(g, u) of one expert row element, following the
// dtype flow of gpu/ir.cpp:1130-1145 under MLX's promotion rules.
//   bf16 flow (BF16 = true), g and u are the bf16-rounded projections:
//     swiglu: h = rbf(rbf(sigmoid(g)) * u)
//     geglu : h = gelu_fp32(g) * u        (fp32: the float scalars promote)
//     mlp silu: h = rbf(u * rbf(sigmoid(u)))       (g unused, u = x.W_up)
//     mlp gelu: h = gelu_fp32(u)
//     mlp relu: h = max(u, 0)
//     mlp leaky_relu_sq: h = (u > 0 ? u : u*slope)^2 in fp32 (slope array is fp32)
//   fp32 flow: the same formulas without rounding.
template <bool BF16>
MXM_HD float mxm_hidden(int expert_type, int activation, float slope, float g, float u) {
  auto R = [](float v) { return BF16 ? mxm_rbf(v) : v; };
  if (expert_type == MXM_EXPERT_SWIGLU) {
    return R(R(mxm_sigmoid(g)) * u);
  }
  if (expert_type == MXM_EXPERT_GEGLU) {
    return mxm_gelu_tanh_sq(g, R(g * g)) * u;
  }
  switch (activation) {
    case MXM_ACT_SILU:
      return R(u * R(mxm_sigmoid(u)));
    case MXM_ACT_GELU:
      return mxm_gelu_tanh_sq(u, R(u * u));
    case MXM_ACT_RELU:
      return u > 0.0f ? u : 0.0f;
    default: {
      const float y = u > 0.0f ? u : u * slope;
      return y * y;
    }
  }
}

// The same activations for the MFMA and int8 epilogues, whose products are
// compared with the CPU restatement within a tolerance (their accumulation
// order differs anyway): exp on the hardware exp2 and the reciprocal on
// v_rcp_f32 (each within about 1 ulp) instead of the exactly specified
// sequences above, and bf16 rounding by the hardware conversion.  The bf16
// roundings of the dtype flow are kept.
// Hardware round-to-nearest-even fp32 -> bf16 (v_cvt_pk_bf16_f32).
__device__ __forceinline__ float mxm_rbf_fast(float f) { return (float)(__bf16)f; }
__device__ __forceinline__ uint16_t mxm_f2bf_fast(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}
// Two values to packed bf16 (lo = bf16(a), hi = bf16(b)), one conversion.
__device__ __forceinline__ uint32_t mxm_pack_bf2_fast(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ float mxm_exp_fast(float x) {
  return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}
__device__ __forceinline__ float mxm_sigmoid_fast(float x) {
  return __builtin_amdgcn_rcpf(1.0f + mxm_exp_fast(-x));
}
__device__ __forceinline__ float mxm_gelu_tanh_sq_fast(float v, float sq) {
  const float d = 0.7978845608f * (v + (0.044715f * v) * sq);
  const float t = mxm_exp_fast(-2.0f * __builtin_fabsf(d));
  const float th = __builtin_copysignf((1.0f - t) * __builtin_amdgcn_rcpf(1.0f + t), d);
  return (0.5f * v) * (1.0f + th);
}
template <bool BF16>
__device__ __forceinline__ float mxm_hidden_fast(int expert_type, int activation, float slope,
                                                 float g, float u) {
  auto R = [](float v) { return BF16 ? mxm_rbf_fast(v) : v; };
  if (expert_type == MXM_EXPERT_SWIGLU) return R(R(mxm_sigmoid_fast(g)) * u);
  if (expert_type == MXM_EXPERT_GEGLU) return mxm_gelu_tanh_sq_fast(g, R(g * g)) * u;
  switch (activation) {
    case MXM_ACT_SILU:
      return R(u * R(mxm_sigmoid_fast(u)));
    case MXM_ACT_GELU:
      return mxm_gelu_tanh_sq_fast(u, R(u * u));
    case MXM_ACT_RELU:
      return u > 0.0f ? u : 0.0f;
    default: {
      const float y = u > 0.0f ? u : u * slope;
      return y * y;
    }
  }
}
