// Gradient clipping by global norm fused with an AdamW step, over one flat
// fp32 parameter buffer, for gfx950.
//
// Replaces the step either side of backward in the reference's train loop
// (packbalance/train/train.py:353-362, profiling/bench_train.py:115-116):
//   torch.nn.utils.clip_grad_norm_(params, max_norm)   then
//   torch.optim.AdamW(params, lr, betas, eps, weight_decay, fused=True).step()
// with uniform hyper-parameters, so the update is element-wise and the whole
// parameter set is one buffer.  The arithmetic is the published AdamW
// (decoupled weight decay) with PyTorch's bias-correction convention:
//   norm  = sqrt(sum g^2);  c = min(max_norm / (norm + 1e-6), 1)   (c = 1 if max_norm <= 0)
//   t    += 1
//   g     = c * grad
//   p     = p - lr*wd*p
//   m     = b1*m + (1-b1)*g;   v = b2*v + (1-b2)*g^2
//   p     = p - (lr / (1 - b1^t)) * m / (sqrt(v) / sqrt(1 - b2^t) + eps)
// and, optionally, the updated p rounded into a bf16/fp16 copy (the weights
// the next step's matmuls read), so no separate cast pass runs.
//
// The gradient may arrive in several slots (grad_slots buffers slot_stride
// elements apart, e.g. one per concurrently run micro-batch): it is their sum,
// which the first pass forms and writes back into slot 0.
//
// Three launches, all streaming with 16-byte non-temporal accesses:
//   1. sq_partial: sums the slots (when more than one) into slot 0, and
//                  per-workgroup sums of g^2 (fixed grid, fixed order);
//   2. prepare:    one workgroup folds the partials in fp64, writes the norm,
//                  advances the device-resident step and stores the per-step
//                  scalars (clip factor, step size, sqrt(1 - b2^t));
//   3. update:     the element-wise step (reads p, g, m, v; writes p, m, v and
//                  the optional copy: 30 bytes per element with a bf16 copy).
// Every scalar that changes per step lives on the device, so the sequence can
// be captured in a HIP graph and replayed.
#include <math.h>

#include "common.hpp"

namespace pb {
namespace {

constexpr int kThreads = 256;
constexpr int kNormWgs = 1024;  // partial sums of the gradient norm
constexpr int kUpdU = 2;        // 4-float groups per thread in the update

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct Scalars {
  float clip;          // factor applied to the gradient
  float step_size;     // lr / (1 - b1^t)
  float bc2_sqrt;      // sqrt(1 - b2^t)
  float pad;
};

// Squared norm of the slot sum, which is written back into slot 0 when there
// are several slots (slot order fixed, so the sum is deterministic).
__global__ __launch_bounds__(kThreads) void sq_partial(float *__restrict__ g, int64_t n, int slots,
                                                       int64_t slot_stride,
                                                       float *__restrict__ partial) {
  __shared__ float red[kThreads / 64];
  const int64_t nvec = n / 4;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  float s0 = 0.f;
  if (slots == 1) {
    float s1 = 0.f;
    int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    for (; i + stride < nvec; i += 2 * stride) {
      const f32x4 a = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(g) + i);
      const f32x4 b = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(g) + i + stride);
      s0 += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
      s1 += b.x * b.x + b.y * b.y + b.z * b.z + b.w * b.w;
    }
    if (i < nvec) {
      const f32x4 a = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(g) + i);
      s0 += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
    }
    s0 += s1;
  } else {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < nvec; i += stride) {
      f32x4 a = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(g) + i);
      for (int sl = 1; sl < slots; ++sl)
        a += __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(g + sl * slot_stride) + i);
      reinterpret_cast<f32x4 *>(g)[i] = a;
      s0 += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
    }
  }
  if (blockIdx.x == 0 && threadIdx.x < n - nvec * 4) {
    const int64_t j = nvec * 4 + threadIdx.x;
    float t = g[j];
    for (int sl = 1; sl < slots; ++sl) t += g[sl * slot_stride + j];
    if (slots > 1) g[j] = t;
    s0 += t * t;
  }
  float s = wave_sum(s0);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) t += red[w];
    partial[blockIdx.x] = t;
  }
}

__global__ __launch_bounds__(kThreads) void prepare(const float *__restrict__ partial, int nparts,
                                                    float max_norm, float lr, float beta1,
                                                    float beta2, float *__restrict__ step,
                                                    float *__restrict__ norm_out,
                                                    Scalars *__restrict__ sc) {
  __shared__ double red[kThreads];
  double s = 0.0;
  for (int p = threadIdx.x; p < nparts; p += kThreads) s += (double)partial[p];
  red[threadIdx.x] = s;
  __syncthreads();
  for (int o = kThreads / 2; o > 0; o >>= 1) {
    if (threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const float norm = (float)sqrt(red[0]);
    if (norm_out) norm_out[0] = norm;
    float clip = 1.0f;
    if (max_norm > 0.f) {
      const float c = max_norm / (norm + 1e-6f);
      clip = c < 1.0f ? c : 1.0f;
    }
    const float t = step[0] + 1.0f;
    step[0] = t;
    Scalars v;
    v.clip = clip;
    v.step_size = (float)((double)lr / (1.0 - pow((double)beta1, (double)t)));
    v.bc2_sqrt = (float)sqrt(1.0 - pow((double)beta2, (double)t));
    v.pad = 0.f;
    sc[0] = v;
  }
}

struct UpdArgs {
  float *p, *m, *v;
  const float *g;
  void *copy;  // nullable
  int copy_dtype;
  int64_t n;
  float lr_wd, beta1, beta2, eps;
  const Scalars *sc;
};

__device__ __forceinline__ void adamw_one(float &p, float &m, float &v, float g, float lr_wd,
                                          float b1, float b2, float eps, float step_size,
                                          float bc2_sqrt) {
  p = p - lr_wd * p;
  m = b1 * m + (1.0f - b1) * g;
  v = b2 * v + (1.0f - b2) * (g * g);
  const float denom = sqrtf(v) / bc2_sqrt + eps;
  p = p - step_size * (m / denom);
}

template <typename C>
__device__ __forceinline__ void store_copy4(void *copy, int64_t i4, const float (&p)[4]) {
  if constexpr (sizeof(C) == 4) {
    __builtin_nontemporal_store(f32x4{p[0], p[1], p[2], p[3]},
                                reinterpret_cast<f32x4 *>(copy) + i4);
  } else {
    C h[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) h[e] = from_f32<C>(p[e]);
    u32x2 raw;
    __builtin_memcpy(&raw, h, 8);
    __builtin_nontemporal_store(raw, reinterpret_cast<u32x2 *>(copy) + i4);
  }
}

// One pass: thread t handles kUpdU float4 groups, kThreads apart.
template <typename C, bool COPY>
__global__ __launch_bounds__(kThreads) void update(UpdArgs a) {
  const Scalars s = *a.sc;
  const int64_t nvec = a.n / 4;
  const int64_t base = (int64_t)blockIdx.x * kThreads * kUpdU + threadIdx.x;
  f32x4 P[kUpdU], G[kUpdU], M[kUpdU], V[kUpdU];
#pragma unroll
  for (int k = 0; k < kUpdU; ++k) {
    const int64_t i = base + (int64_t)k * kThreads;
    if (i < nvec) {
      P[k] = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(a.p) + i);
      G[k] = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(a.g) + i);
      M[k] = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(a.m) + i);
      V[k] = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(a.v) + i);
    }
  }
#pragma unroll
  for (int k = 0; k < kUpdU; ++k) {
    const int64_t i = base + (int64_t)k * kThreads;
    if (i < nvec) {
      float p[4] = {P[k].x, P[k].y, P[k].z, P[k].w};
      float m[4] = {M[k].x, M[k].y, M[k].z, M[k].w};
      float v[4] = {V[k].x, V[k].y, V[k].z, V[k].w};
      const float g[4] = {G[k].x, G[k].y, G[k].z, G[k].w};
#pragma unroll
      for (int e = 0; e < 4; ++e)
        adamw_one(p[e], m[e], v[e], g[e] * s.clip, a.lr_wd, a.beta1, a.beta2, a.eps, s.step_size,
                  s.bc2_sqrt);
      __builtin_nontemporal_store(f32x4{p[0], p[1], p[2], p[3]},
                                  reinterpret_cast<f32x4 *>(a.p) + i);
      __builtin_nontemporal_store(f32x4{m[0], m[1], m[2], m[3]},
                                  reinterpret_cast<f32x4 *>(a.m) + i);
      __builtin_nontemporal_store(f32x4{v[0], v[1], v[2], v[3]},
                                  reinterpret_cast<f32x4 *>(a.v) + i);
      if constexpr (COPY) store_copy4<C>(a.copy, i, p);
    }
  }
  // Tail (n % 4 elements): the first threads of workgroup 0.
  if (blockIdx.x == 0 && threadIdx.x < a.n - nvec * 4) {
    const int64_t j = nvec * 4 + threadIdx.x;
    float p = a.p[j], m = a.m[j], v = a.v[j];
    adamw_one(p, m, v, a.g[j] * s.clip, a.lr_wd, a.beta1, a.beta2, a.eps, s.step_size,
              s.bc2_sqrt);
    a.p[j] = p;
    a.m[j] = m;
    a.v[j] = v;
    if constexpr (COPY) static_cast<C *>(a.copy)[j] = from_f32<C>(p);
  }
}

bool al16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace pb

extern "C" int64_t pb_clip_adamw_workspace_bytes(int64_t n) {
  (void)n;
  return (int64_t)(pb::kNormWgs * sizeof(float) + 256);
}

extern "C" int pb_clip_adamw_step(float *param, float *grad, int grad_slots,
                                  int64_t grad_slot_stride, float *exp_avg, float *exp_avg_sq,
                                  void *param_copy, int copy_dtype, int64_t n, float lr,
                                  float beta1, float beta2, float eps, float weight_decay,
                                  float max_grad_norm, float *step, float *grad_norm_out,
                                  void *workspace, void *stream) {
  using namespace pb;
  clear_error();
  PB_CHECK_ARG(param && grad && exp_avg && exp_avg_sq && step && workspace,
               "pb_clip_adamw_step: null argument");
  PB_CHECK_ARG(n >= 0, "pb_clip_adamw_step: negative size");
  PB_CHECK_ARG(!param_copy || valid_dtype(copy_dtype), "pb_clip_adamw_step: bad copy dtype");
  PB_CHECK_ARG(al16(param) && al16(grad) && al16(exp_avg) && al16(exp_avg_sq) &&
                   (!param_copy || (reinterpret_cast<uintptr_t>(param_copy) & 7) == 0) &&
                   al16(workspace),
               "pb_clip_adamw_step: buffers must be 16-byte aligned (the copy 8-byte aligned)");
  PB_CHECK_ARG(beta1 >= 0.f && beta1 < 1.f && beta2 >= 0.f && beta2 < 1.f && eps > 0.f,
               "pb_clip_adamw_step: bad hyper-parameters");
  PB_CHECK_ARG(grad_slots >= 1 && grad_slots <= 64 &&
                   (grad_slots == 1 || (grad_slot_stride >= n && grad_slot_stride % 4 == 0)),
               "pb_clip_adamw_step: bad gradient slots (count 1..64, stride >= n, %% 4 == 0)");
  // Keeps the update grid (n / 4 / 512 workgroups) below 2^31.
  PB_CHECK_SUPPORTED(n < (1LL << 38), "pb_clip_adamw_step: too large");
  hipStream_t st = as_stream(stream);
  float *partial = static_cast<float *>(workspace);
  Scalars *sc = reinterpret_cast<Scalars *>(static_cast<char *>(workspace) + kNormWgs * sizeof(float));
  hipLaunchKernelGGL(sq_partial, dim3(kNormWgs), dim3(kThreads), 0, st, grad, n, grad_slots,
                     grad_slot_stride, partial);
  hipLaunchKernelGGL(prepare, dim3(1), dim3(kThreads), 0, st, partial, kNormWgs, max_grad_norm, lr,
                     beta1, beta2, step, grad_norm_out, sc);
  int rc = launch_status("pb_clip_adamw_step(norm)");
  if (rc) return rc;
  if (n == 0) return PB_OK;
  UpdArgs a;
  a.p = param; a.m = exp_avg; a.v = exp_avg_sq; a.g = grad;
  a.copy = param_copy;
  a.copy_dtype = copy_dtype;
  a.n = n;
  a.lr_wd = lr * weight_decay;
  a.beta1 = beta1; a.beta2 = beta2; a.eps = eps;
  a.sc = sc;
  const int64_t per_wg = (int64_t)kThreads * kUpdU;
  const int64_t nvec = n / 4;
  dim3 grid((unsigned)((nvec + per_wg - 1) / per_wg > 0 ? (nvec + per_wg - 1) / per_wg : 1));
  if (!param_copy)
    hipLaunchKernelGGL((update<float, false>), grid, dim3(kThreads), 0, st, a);
  else if (copy_dtype == PB_BF16)
    hipLaunchKernelGGL((update<bf16_t, true>), grid, dim3(kThreads), 0, st, a);
  else if (copy_dtype == PB_F16)
    hipLaunchKernelGGL((update<f16_t, true>), grid, dim3(kThreads), 0, st, a);
  else
    hipLaunchKernelGGL((update<float, true>), grid, dim3(kThreads), 0, st, a);
  return launch_status("pb_clip_adamw_step(update)");
}
