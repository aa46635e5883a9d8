// AdamW / Adam step of libpanmuon: the half of PAN 2's optimizer step that
// pan/optim/muon.py:155-164 builds as torch.optim.AdamW(fused=True) over the
// params Muon does not take (embeddings, norms, modulation, heads). One launch
// walks every tensor of a call in chunks of kAdamChunk elements, with the
// per-element arithmetic of torch's Adam (TORCH/optim/adam.py:347-549,
// _single_tensor_adam) carried out in fp32 and each result rounded once to its
// storage dtype, as torch's fused kernel (torch._fused_adamw_, reached from
// TORCH/optim/adam.py:878) does. HBM-bound: fp32 state moves 28 bytes per
// element (param, exp_avg, exp_avg_sq read and written, grad read).
#pragma once

namespace pm {

constexpr int kAdamChunk = 8192;  // elements per block: 4 passes of 256 threads x 8

struct AdamDesc {
  void* p;
  void* g;     // written back only when a grad scale unscales it
  void* m;     // exp_avg
  void* v;     // exp_avg_sq
  void* vmax;  // max_exp_avg_sq (amsgrad), else null
  float* step;
  int64_t n;
  int32_t p_dt, g_dt, m_dt, v_dt;
};

struct AdamArgs {
  const AdamDesc* descs;
  const int32_t* prefix;  // n+1 prefix sums of chunks per tensor
  int32_t n;
  double b1d, b2d;        // beta1, beta2 as the Python floats the bias corrections use
  float beta2;            // as an fp32 scalar (exp_avg_sq.mul_(beta2))
  float w1, w2;           // 1 - beta1, 1 - beta2, rounded from double as torch's scalars are
  float eps;
  float wd;               // weight decay as an fp32 scalar
  double wdd;             // and as the Python float (host-lr decoupled factor)
  int32_t amsgrad, maximize, decoupled;
  const float* lr_dev;    // device lr, or null (then lr_host)
  double lr_host;
  const float* grad_scale;  // grads are divided by *grad_scale and stored unscaled, or null
  const float* found_inf;   // skip the update when *found_inf != 0, or null
};

// Eight consecutive elements of an f32, bf16 or f16 tensor as fp32 (f32 and
// bf16 through the prologue's load8 / store8; f16 here, 16-byte vectors when
// aligned). f16 results are rounded to nearest even, as torch's fused kernel
// stores its fp32 results.
__device__ __forceinline__ void adam_load8(const void* base, int32_t dt, int64_t off, bool vec, int valid,
                                           float (&v)[8]) {
  if (dt != DT_F16) {
    load8(base, dt, off, vec, true, valid, v);
    return;
  }
  const _Float16* h = (const _Float16*)base + off;
  if (vec && valid >= 8) {
    typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
    const f16x8 a = *(const f16x8*)h;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (float)a[e];
    return;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = e < valid ? (float)h[e] : 0.0f;
}

__device__ __forceinline__ void adam_store8(void* base, int32_t dt, int64_t off, bool vec, int valid,
                                            const float (&v)[8]) {
  if (dt != DT_F16) {
    store8(base, dt, off, vec, valid, v);
    return;
  }
  _Float16* h = (_Float16*)base + off;
  if (vec && valid >= 8) {
    typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
    f16x8 a;
#pragma unroll
    for (int e = 0; e < 8; ++e) a[e] = (_Float16)v[e];
    *(f16x8*)h = a;
    return;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (e < valid) h[e] = (_Float16)v[e];
}

__device__ __forceinline__ bool adam_vec_ok(const void* base, int32_t dt) {
  return (uintptr_t)base % 16 == 0 && (dt == DT_F32 || dt == DT_BF16 || dt == DT_F16);
}

// step += 1 for every tensor (TORCH/optim/adam.py:877), less found_inf, which
// torch subtracts again after a skipped update (:895-898).
__global__ __launch_bounds__(kThreads) void pm_adam_count_kernel(const AdamDesc* descs, int n,
                                                                 const float* found_inf) {
  const int i = blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  const float inc = found_inf ? 1.0f - *found_inf : 1.0f;
  *descs[i].step = *descs[i].step + inc;
}

// torch.maximum: NaN if either operand is NaN.
__device__ __forceinline__ float nan_max(float a, float b) { return (a != a || b != b) ? a + b : fmaxf(a, b); }

// ATen's scalar lerp: self + w (end - self) for |w| < 0.5, else end - (end - self)(1 - w).
__device__ __forceinline__ float torch_lerp(float self, float end, float w) {
#pragma clang fp contract(off)
  return fabsf(w) < 0.5f ? self + w * (end - self) : end - (end - self) * (1.0f - w);
}

__global__ __launch_bounds__(kThreads) void pm_adam_kernel(AdamArgs a) {
#pragma clang fp contract(off)
  if (a.found_inf && *a.found_inf != 0.0f) return;
  const int t = blockIdx.x;
  const int ti = find_matrix(a.prefix, a.n, t);
  const AdamDesc& d = a.descs[ti];
  const int64_t base = (int64_t)(t - a.prefix[ti]) * kAdamChunk;
  // per-tensor scalars (TORCH/optim/adam.py:529-536, Python floats = double):
  // bias corrections, step size, sqrt of the second correction
  const double lr = a.lr_dev ? (double)*a.lr_dev : a.lr_host;
  const double step = (double)*d.step;
  const double bc1 = 1.0 - pow(a.b1d, step);
  const double bc2 = 1.0 - pow(a.b2d, step);
  const float neg_step = (float)(-(lr / bc1));
  const float bc2_sqrt = (float)sqrt(bc2);
  // decoupled decay: param.mul_(1 - lr * weight_decay) (:419)
  const float wdf = a.lr_dev ? 1.0f - (float)lr * a.wd : (float)(1.0 - lr * a.wdd);
  const float scale = a.grad_scale ? *a.grad_scale : 1.0f;
  const bool pv = adam_vec_ok(d.p, d.p_dt), gv = adam_vec_ok(d.g, d.g_dt), mv = adam_vec_ok(d.m, d.m_dt),
             vv = adam_vec_ok(d.v, d.v_dt), xv = a.amsgrad && adam_vec_ok(d.vmax, d.v_dt);
#pragma unroll 1
  for (int it = 0; it < kAdamChunk / (kThreads * 8); ++it) {
    const int64_t off = base + ((int64_t)it * kThreads + threadIdx.x) * 8;
    if (off >= d.n) break;
    const int valid = d.n - off >= 8 ? 8 : (int)(d.n - off);
    float p[8], g[8], m[8], v[8], x[8];
    adam_load8(d.p, d.p_dt, off, pv, valid, p);
    adam_load8(d.g, d.g_dt, off, gv, valid, g);
    adam_load8(d.m, d.m_dt, off, mv, valid, m);
    adam_load8(d.v, d.v_dt, off, vv, valid, v);
    if (a.amsgrad) adam_load8(d.vmax, d.v_dt, off, xv, valid, x);
    if (a.grad_scale) {
      // the fused kernel leaves the grads unscaled (a GradScaler's unscale_)
#pragma unroll
      for (int e = 0; e < 8; ++e) g[e] = g[e] / scale;
      adam_store8(d.g, d.g_dt, off, gv, valid, g);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float gr0 = a.maximize ? -g[e] : g[e];
      float gr = gr0;
      float pe = p[e];
      if (a.wd != 0.0f) {
        if (a.decoupled) pe = pe * wdf;
        else gr = gr + a.wd * pe;  // grad.add(param, alpha=weight_decay) (:429)
      }
      m[e] = torch_lerp(m[e], gr, a.w1);            // exp_avg.lerp_(grad, 1 - beta1) (:457)
      v[e] = v[e] * a.beta2 + (a.w2 * gr) * gr;     // exp_avg_sq.mul_(beta2).addcmul_(grad, grad, 1 - beta2) (:476)
      float vh = v[e];
      if (a.amsgrad) {
        x[e] = nan_max(x[e], v[e]);                   // torch.maximum(max_exp_avg_sq, exp_avg_sq) (:540)
        vh = x[e];
      }
      const float denom = sqrtf(vh) / bc2_sqrt + a.eps;  // (:541-545)
      p[e] = pe + neg_step * (m[e] / denom);             // param.addcdiv_(exp_avg, denom, value=-step_size) (:547)
    }
    adam_store8(d.p, d.p_dt, off, pv, valid, p);
    adam_store8(d.m, d.m_dt, off, mv, valid, m);
    adam_store8(d.v, d.v_dt, off, vv, valid, v);
    if (a.amsgrad) adam_store8(d.vmax, d.v_dt, off, xv, valid, x);
  }
}

}  // namespace pm
