// tl_norm_act.hip -- the read-side neighbours of attention: RMSNorm, fused
// residual add + RMSNorm, LayerNorm (layernorm_kernels.cu:28-147) and the
// gated activations silu / gelu / gelu_tanh _and_mul
// (activation_kernels.cu:57-132), for gfx950.
//
// Intended semantics, in fp32 (the reference's, less its defect D4: its
// block reduction leaves the total in warp 0 only, so every other warp
// normalises with its own partial sum):
//   rms_norm:    out = T(x * rsqrt(sum(x^2)/H + eps) * w)
//   fused_add:   r = res + x; res = T(r); sum over r (unrounded);
//                out = T(float(res) * rsqrt(...) * w)
//   layer_norm:  mean, var = sum((x - mean)^2)/H (two passes),
//                out = T((x - mean) * rsqrt(var + eps) * w + b)
//   act_and_mul: out = T(float(T(act(gate))) * up): the activation is
//                rounded to T first, as the reference's act() returns T
//   silu(x) = x / (1 + exp(-x)) (hardware exp / reciprocal for f16 / bf16,
//   below their rounding); gelu(x) = 0.5 x (1 + erf(x / sqrt 2));
//   gelu_tanh(x) = 0.5 x (1 + tanh(0.79788456 (x + 0.044715 x^3))).
// One workgroup per row for the norms (256 threads, the row strided over
// them, the total reduced over the workgroup); the activations are one
// element per thread.  All of them are HBM-bound at serving sizes.
#include "tl_device.hpp"
#include "tl_internal.hpp"

namespace tl {

namespace {

constexpr int kNormThreads = 256;

// Sum over the workgroup, returned to every thread.
__device__ __forceinline__ float block_sum(float v, float* s_part) {
#pragma unroll
  for (int o = kWave / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o, kWave);
  const int wave = threadIdx.x / kWave;
  __syncthreads();                                   // s_part free from a previous use
  if (threadIdx.x % kWave == 0) s_part[wave] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < kNormThreads / kWave; ++w) t += s_part[w];
  return t;
}

template <Kind K>
__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(void* __restrict__ out, void* __restrict__ residual,
                                                                const void* __restrict__ x,
                                                                const void* __restrict__ w, int hidden, float eps,
                                                                bool fused_add) {
  __shared__ float s_part[kNormThreads / kWave];
  const int64_t base = (int64_t)blockIdx.x * hidden;
  float ss = 0.f;
  for (int i = threadIdx.x; i < hidden; i += kNormThreads) {
    float v = load_scalar<K>(x, base + i);
    if (fused_add) {
      v += load_scalar<K>(residual, base + i);
      store_scalar<K>(residual, base + i, v);
    }
    ss = __builtin_fmaf(v, v, ss);
  }
  const float inv = 1.0f / __builtin_sqrtf(block_sum(ss, s_part) / (float)hidden + eps);
  const void* src = fused_add ? residual : x;
  for (int i = threadIdx.x; i < hidden; i += kNormThreads)
    store_scalar<K>(out, base + i, load_scalar<K>(src, base + i) * inv * load_scalar<K>(w, i));
}

// Round to the storage type and back (identity for f32).
template <Kind K> __device__ __forceinline__ float round_to(float v);
template <> __device__ __forceinline__ float round_to<Kind::F32>(float v) { return v; }
template <> __device__ __forceinline__ float round_to<Kind::F16>(float v) { return f16_to_f32(f32_to_f16(v)); }
template <> __device__ __forceinline__ float round_to<Kind::BF16>(float v) { return bf16_to_f32(f32_to_bf16(v)); }

template <Kind K> __device__ __forceinline__ void unpack8(const u32x4& c, float (&f)[8]) {
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint16_t b = (uint16_t)(w[j / 2] >> (16 * (j & 1)));
    f[j] = K == Kind::F16 ? f16_to_f32(b) : bf16_to_f32(b);
  }
}
template <Kind K> __device__ __forceinline__ u32x4 pack8(const float (&f)[8]) {
  uint32_t w[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint16_t lo = K == Kind::F16 ? f32_to_f16(f[2 * k]) : f32_to_bf16(f[2 * k]);
    const uint16_t hi = K == Kind::F16 ? f32_to_f16(f[2 * k + 1]) : f32_to_bf16(f[2 * k + 1]);
    w[k] = (uint32_t)lo | ((uint32_t)hi << 16);
  }
  return u32x4{w[0], w[1], w[2], w[3]};
}

// 2-byte rows of up to C x 2048 elements (C 16-byte chunks per thread),
// held in registers between the two passes.
template <Kind K, int C>
__global__ __launch_bounds__(kNormThreads) void rms_norm_vec_kernel(void* __restrict__ out, void* __restrict__ residual,
                                                                    const void* __restrict__ x,
                                                                    const void* __restrict__ w, int hidden,
                                                                    float eps, bool fused_add) {
  __shared__ float s_part[kNormThreads / kWave];
  const int64_t base = (int64_t)blockIdx.x * hidden;
  float v[C][8];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int i0 = (c * kNormThreads + (int)threadIdx.x) * 8;
    if (i0 >= hidden) break;
    unpack8<K>(load16((const uint16_t*)x + base + i0), v[c]);
    if (fused_add) {
      float r[8];
      unpack8<K>(load16((const uint16_t*)residual + base + i0), r);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float sum = v[c][j] + r[j];
        ss = __builtin_fmaf(sum, sum, ss);
        v[c][j] = round_to<K>(sum);
      }
      *reinterpret_cast<u32x4*>((uint16_t*)residual + base + i0) = pack8<K>(v[c]);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) ss = __builtin_fmaf(v[c][j], v[c][j], ss);
    }
  }
  const float inv = 1.0f / __builtin_sqrtf(block_sum(ss, s_part) / (float)hidden + eps);
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int i0 = (c * kNormThreads + (int)threadIdx.x) * 8;
    if (i0 >= hidden) break;
    float wf[8], o[8];
    unpack8<K>(load16((const uint16_t*)w + i0), wf);
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = v[c][j] * inv * wf[j];
    *reinterpret_cast<u32x4*>((uint16_t*)out + base + i0) = pack8<K>(o);
  }
}

template <Kind K>
__global__ __launch_bounds__(kNormThreads) void layer_norm_kernel(void* __restrict__ out, const void* __restrict__ x,
                                                                  const void* __restrict__ w,
                                                                  const void* __restrict__ b, int hidden,
                                                                  float eps) {
  __shared__ float s_part[kNormThreads / kWave];
  const int64_t base = (int64_t)blockIdx.x * hidden;
  float s = 0.f;
  for (int i = threadIdx.x; i < hidden; i += kNormThreads) s += load_scalar<K>(x, base + i);
  const float mean = block_sum(s, s_part) / (float)hidden;
  float var = 0.f;
  for (int i = threadIdx.x; i < hidden; i += kNormThreads) {
    const float d = load_scalar<K>(x, base + i) - mean;
    var = __builtin_fmaf(d, d, var);
  }
  const float inv = 1.0f / __builtin_sqrtf(block_sum(var, s_part) / (float)hidden + eps);
  for (int i = threadIdx.x; i < hidden; i += kNormThreads) {
    const float nrm = (load_scalar<K>(x, base + i) - mean) * inv;
    store_scalar<K>(out, base + i, __builtin_fmaf(nrm, load_scalar<K>(w, i), load_scalar<K>(b, i)));
  }
}

template <Kind K, int ACT>
__global__ __launch_bounds__(256) void act_and_mul_kernel(void* __restrict__ out, const void* __restrict__ gate,
                                                          const void* __restrict__ up, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float g = load_scalar<K>(gate, i);
  float a;
  if constexpr (ACT == 0) {
    a = K == Kind::F32 ? g / (1.f + expf(-g)) : g * __builtin_amdgcn_rcpf(1.f + __expf(-g));
  } else if constexpr (ACT == 1) {
    a = 0.5f * g * (1.f + erff(g * 0.70710678118f));
  } else {
    const float c = 0.79788456f * (g + 0.044715f * g * g * g);
    a = 0.5f * g * (1.f + tanhf(c));
  }
  store_scalar<K>(out, i, round_to<K>(a) * load_scalar<K>(up, i));
}

// 2-byte types, 8 elements (16 bytes) per thread.  exp and the division
// run at hardware precision (v_exp_f32, v_rcp_f32: an fp32 ulp or two, far
// below the rounding to f16 / bf16; the reference builds with
// --use_fast_math, which does the same).
template <Kind K, int ACT>
__global__ __launch_bounds__(256) void act_and_mul_vec_kernel(void* __restrict__ out, const void* __restrict__ gate,
                                                              const void* __restrict__ up, int64_t n8) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n8) return;
  const u32x4 gw = load16((const uint16_t*)gate + 8 * i), uw = load16((const uint16_t*)up + 8 * i);
  const uint32_t gs[4] = {gw.x, gw.y, gw.z, gw.w}, us[4] = {uw.x, uw.y, uw.z, uw.w};
  uint32_t o[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    uint32_t pair = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint16_t gb = (uint16_t)(gs[k] >> (16 * h)), ub = (uint16_t)(us[k] >> (16 * h));
      const float g = K == Kind::F16 ? f16_to_f32(gb) : bf16_to_f32(gb);
      const float u = K == Kind::F16 ? f16_to_f32(ub) : bf16_to_f32(ub);
      float a;
      if constexpr (ACT == 0) {
        a = g * __builtin_amdgcn_rcpf(1.f + __expf(-g));
      } else if constexpr (ACT == 1) {
        a = 0.5f * g * (1.f + erff(g * 0.70710678118f));
      } else {
        const float c = 0.79788456f * (g + 0.044715f * g * g * g);
        a = 0.5f * g * (1.f + tanhf(c));
      }
      const float v = round_to<K>(a) * u;
      const uint16_t ob = K == Kind::F16 ? f32_to_f16(v) : f32_to_bf16(v);
      pair |= (uint32_t)ob << (16 * h);
    }
    o[k] = pair;
  }
  *reinterpret_cast<u32x4*>((uint16_t*)out + 8 * i) = u32x4{o[0], o[1], o[2], o[3]};
}

template <Kind K>
int launch_act_typed(void* out, const void* gate, const void* up, int64_t n, int act, hipStream_t stream) {
  const auto al = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  int64_t done = 0;
  if constexpr (K != Kind::F32) {
    if (al(out) && al(gate) && al(up) && n >= 8) {
      const int64_t n8 = n / 8;
      const dim3 grid((unsigned)((n8 + 255) / 256));
      if (act == 0) hipLaunchKernelGGL((act_and_mul_vec_kernel<K, 0>), grid, dim3(256), 0, stream, out, gate, up, n8);
      else if (act == 1) hipLaunchKernelGGL((act_and_mul_vec_kernel<K, 1>), grid, dim3(256), 0, stream, out, gate, up, n8);
      else hipLaunchKernelGGL((act_and_mul_vec_kernel<K, 2>), grid, dim3(256), 0, stream, out, gate, up, n8);
      done = n8 * 8;
    }
  }
  const int64_t rest = n - done;
  if (rest > 0) {
    const int64_t e = K == Kind::F32 ? 4 : 2;
    void* o = (char*)out + done * e;
    const void* g = (const char*)gate + done * e;
    const void* u = (const char*)up + done * e;
    const dim3 grid((unsigned)((rest + 255) / 256));
    if (act == 0) hipLaunchKernelGGL((act_and_mul_kernel<K, 0>), grid, dim3(256), 0, stream, o, g, u, rest);
    else if (act == 1) hipLaunchKernelGGL((act_and_mul_kernel<K, 1>), grid, dim3(256), 0, stream, o, g, u, rest);
    else hipLaunchKernelGGL((act_and_mul_kernel<K, 2>), grid, dim3(256), 0, stream, o, g, u, rest);
  }
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

}  // namespace

int launch_rms_norm(void* out, void* residual, const void* x, const void* w, int rows, int hidden, float eps,
                    int dtype, hipStream_t stream) {
  if (rows == 0) return 0;
  const bool fused = residual != nullptr;
  const Kind k = (Kind)dtype;
  const auto al = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  const int chunks = (hidden + kNormThreads * 8 - 1) / (kNormThreads * 8);
  if ((k == Kind::F16 || k == Kind::BF16) && hidden % 8 == 0 && chunks <= 4 && al(out) && al(x) && al(w) &&
      (!fused || al(residual))) {
#define TL_RMS_VEC(KK, C)                                                                                      \
  hipLaunchKernelGGL((rms_norm_vec_kernel<KK, C>), dim3(rows), dim3(kNormThreads), 0, stream, out, residual, x, \
                     w, hidden, eps, fused)
    if (k == Kind::F16) {
      if (chunks == 1) TL_RMS_VEC(Kind::F16, 1); else if (chunks == 2) TL_RMS_VEC(Kind::F16, 2);
      else if (chunks == 3) TL_RMS_VEC(Kind::F16, 3); else TL_RMS_VEC(Kind::F16, 4);
    } else {
      if (chunks == 1) TL_RMS_VEC(Kind::BF16, 1); else if (chunks == 2) TL_RMS_VEC(Kind::BF16, 2);
      else if (chunks == 3) TL_RMS_VEC(Kind::BF16, 3); else TL_RMS_VEC(Kind::BF16, 4);
    }
#undef TL_RMS_VEC
    return hipGetLastError() == hipSuccess ? 0 : 5;
  }
  if (k == Kind::F16)
    hipLaunchKernelGGL(rms_norm_kernel<Kind::F16>, dim3(rows), dim3(kNormThreads), 0, stream, out, residual, x, w,
                       hidden, eps, fused);
  else if (k == Kind::BF16)
    hipLaunchKernelGGL(rms_norm_kernel<Kind::BF16>, dim3(rows), dim3(kNormThreads), 0, stream, out, residual, x,
                       w, hidden, eps, fused);
  else if (k == Kind::F32)
    hipLaunchKernelGGL(rms_norm_kernel<Kind::F32>, dim3(rows), dim3(kNormThreads), 0, stream, out, residual, x, w,
                       hidden, eps, fused);
  else
    return 3;
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

int launch_layer_norm(void* out, const void* x, const void* w, const void* b, int rows, int hidden, float eps,
                      int dtype, hipStream_t stream) {
  if (rows == 0) return 0;
  const Kind k = (Kind)dtype;
  if (k == Kind::F16)
    hipLaunchKernelGGL(layer_norm_kernel<Kind::F16>, dim3(rows), dim3(kNormThreads), 0, stream, out, x, w, b,
                       hidden, eps);
  else if (k == Kind::BF16)
    hipLaunchKernelGGL(layer_norm_kernel<Kind::BF16>, dim3(rows), dim3(kNormThreads), 0, stream, out, x, w, b,
                       hidden, eps);
  else if (k == Kind::F32)
    hipLaunchKernelGGL(layer_norm_kernel<Kind::F32>, dim3(rows), dim3(kNormThreads), 0, stream, out, x, w, b,
                       hidden, eps);
  else
    return 3;
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

int launch_act_and_mul(void* out, const void* gate, const void* up, int64_t n, int act, int dtype,
                       hipStream_t stream) {
  if (n == 0) return 0;
  const Kind k = (Kind)dtype;
  if (k == Kind::F16) return launch_act_typed<Kind::F16>(out, gate, up, n, act, stream);
  if (k == Kind::BF16) return launch_act_typed<Kind::BF16>(out, gate, up, n, act, stream);
  if (k == Kind::F32) return launch_act_typed<Kind::F32>(out, gate, up, n, act, stream);
  return 3;
}

}  // namespace tl
