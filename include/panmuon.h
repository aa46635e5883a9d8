/*
 * panmuon.h — C ABI of the MI355X (gfx950) Muon optimizer library, libpanmuon.so.
 *
 * The library replaces the device work behind PAN 2's patched Muon step:
 *   - the per-parameter loop of pan/optim/patch_muon.py:146-171
 *     (momentum -> Newton–Schulz -> parameter step), and
 *   - the Triton/quack kernels it calls (pan/optim/muon_triton.py,
 *     quack gemm_symmetric, gemm_symmetric_out and gemm_out at pan/optim/patch_muon.py:310-333).
 *
 * Conventions (mirroring the reference):
 *   - Parameters and momentum buffers belong to the caller and are updated in
 *     place; every other buffer lives in a caller-provided device workspace.
 *     No entry point allocates device memory.
 *   - All device work is enqueued on the caller's stream (a hipStream_t passed
 *     as void*); nothing synchronises the host.
 *   - Return codes: 0 on success, a negative PM_E* value on failure; the text
 *     of the last failure on the calling thread is pm_last_error().
 *   - Matrices are row-major with unit column stride and a row stride ("ld")
 *     in elements.
 *
 * Newton–Schulz comes in two organisations (pm_hparams.ns_form):
 *   PM_NS_STANDARD: the quintic of torch.optim._muon
 *     (_zeropower_via_newtonschulz, torch/optim/_muon.py:31-70): per
 *     iteration A = X Xᵀ, B = b A + c A², X <- a X + B X.
 *   PM_NS_GRAM: PAN 2's production form (_gram_newtonschulz_local,
 *     pan/optim/patch_muon.py:275-334): the iteration runs on the gram
 *     R = X Xᵀ and accumulates the polynomial Q, so only two grams and two
 *     applications X <- Q X touch the full matrix (X is re-grammed at
 *     iteration 2). Equal to the standard form in exact arithmetic.
 * X is oriented so that its short side is contracted. Operands are bf16,
 * accumulation fp32, and every GEMM output is rounded to bf16 where the
 * reference rounds it.
 */
#ifndef PANMUON_H
#define PANMUON_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PM_ABI_VERSION 2

/* Element types accepted for params, grads, momentum buffers and updates.
 * PM_DTYPE_F16 is accepted by pm_adam_step only, as torch's fused Adam takes
 * fp16 params and state (torch/optim/adam.py:803-898); the Muon entry points
 * take f32 and bf16. */
enum pm_dtype {
  PM_DTYPE_F32 = 0,
  PM_DTYPE_BF16 = 1,
  PM_DTYPE_F16 = 2
};

/* pm_hparams.ns_form */
enum pm_ns_form {
  PM_NS_STANDARD = 0,
  PM_NS_GRAM = 1
};

enum pm_status {
  PM_OK = 0,
  PM_EINVAL = -1,       /* bad argument (null pointer, bad shape, bad stride) */
  PM_EDTYPE = -2,       /* unsupported dtype */
  PM_EWORKSPACE = -3,   /* workspace too small */
  PM_EHIP = -4,         /* a HIP runtime call failed */
  PM_EUNSUPPORTED = -5  /* valid request this build does not implement */
};

/*
 * One Muon parameter (a 2-D weight, or one row block of a chunked weight).
 * param/grad/momentum are rows x cols with their own row strides.
 * adj_ratio is the shape factor of torch.optim._muon._adjust_lr
 * (torch/optim/_muon.py:73-84): adjusted_lr = lr * adj_ratio. It is computed
 * by the caller from the shape the reference passes (the chunk shape for
 * chunked params, pan/optim/patch_muon.py:142).
 */
typedef struct pm_matrix {
  void* param;
  const void* grad;
  void* momentum;
  int64_t rows;
  int64_t cols;
  int64_t param_ld;
  int64_t grad_ld;
  int64_t momentum_ld;
  int32_t param_dtype;
  int32_t grad_dtype;
  int32_t momentum_dtype;
  int32_t reserved;
  double adj_ratio;
} pm_matrix;

/* One matrix for the Newton–Schulz-only entry point: out = NS(in), bf16. */
typedef struct pm_ns_matrix {
  const void* in;
  void* out;
  int64_t rows;
  int64_t cols;
  int64_t in_ld;
  int64_t out_ld;
  int32_t in_dtype;
  int32_t reserved;
} pm_ns_matrix;

/*
 * Hyper-parameters shared by every matrix of one call. They are the keyword
 * arguments of torch.optim._muon._single_tensor_muon
 * (pan/optim/patch_muon.py:44-58): momentum, nesterov, ns_coefficients,
 * ns_steps, eps, weight_decay.
 *   coeffs: NULL to use (a, b, c) for every iteration, or a host array of
 *           ns_steps triples (a, b, c) — one per iteration.
 *   ns_form: PM_NS_STANDARD (torch's quintic) or PM_NS_GRAM (PAN 2's gram
 *           form, pan/optim/patch_muon.py:275-334).
 *   workspace_limit: upper bound in bytes on the workspace pm_workspace_bytes
 *           asks for (0 = library default); matrices are then processed in
 *           groups that fit.
 */
typedef struct pm_hparams {
  float momentum;
  int32_t nesterov;
  int32_t ns_steps;
  float eps;
  double weight_decay;
  float a;
  float b;
  float c;
  int32_t ns_form;
  const float* coeffs;
  uint64_t workspace_limit;
} pm_hparams;

/* ABI version of the loaded library (PM_ABI_VERSION). */
int pm_abi_version(void);

/* Text of the last failure on the calling thread ("" if none). */
const char* pm_last_error(void);

/*
 * Workspace needed by pm_muon_step for these matrices. Replaces the torch
 * caching-allocator temporaries of pan/optim/muon_triton.py:98 and
 * pan/optim/patch_muon.py:305-308. Returns 0 and sets pm_last_error on a bad
 * argument.
 */
size_t pm_workspace_bytes(const pm_matrix* mats, int n, const pm_hparams* hp);

/*
 * One Muon step over n matrices, in place. Replaces the single-GPU per-param
 * loop of PAN 2's _single_tensor_muon (pan/optim/patch_muon.py:146-171):
 *   buf <- mu*buf + (1-mu)*g;  u <- (1-mu)*g + mu*buf   (nesterov; else u = buf)
 *                                    (pan/optim/muon_triton.py:44-48)
 *   O   <- NS(u)                     (torch/optim/_muon.py:55-69)
 *   p   <- p*(1 - lr*wd) - lr*adj_ratio*O
 *                                    (pan/optim/muon_triton.py:130-131,188-190)
 * lr is read from lr_dev (a device float, the reference's tensor lr path,
 * pan/optim/muon_triton.py:152-159) when it is not NULL, else lr_host.
 * On a stream under graph capture the descriptor table goes in as kernel
 * arguments rather than as a copy from the library's staging buffers, so a
 * captured call replays correctly while the workspace it was given stays
 * allocated (the same holds for pm_newton_schulz and pm_adam_step).
 */
int pm_muon_step(const pm_matrix* mats, int n, const pm_hparams* hp,
                 const float* lr_dev, double lr_host,
                 void* workspace, size_t workspace_bytes, void* stream);

/*
 * pm_muon_step without a caller workspace and without any allocation. No
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory while they step (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). Same arguments and results as
 * pm_muon_step; the workspace is a static device array of
 * PM_NOALLOC_SCRATCH_BYTES that every GPU the library runs on holds until the
 * process ends, and the descriptor tables travel as kernel arguments. A
 * matrix whose own workspace exceeds the scratch fails with PM_EWORKSPACE
 * before anything is enqueued. Calls that overlap on one GPU (other threads,
 * other streams) share its scratch and race; serialise them. The first call
 * on a device looks the scratch up (hipGetSymbolAddress), which may load the
 * code object: make one call outside capture before capturing a graph. A
 * captured call enqueues kernel launches only (no memset or copy nodes); its
 * replays re-read lr_dev on the device and step the same tensors.
 */
#define PM_NOALLOC_SCRATCH_BYTES (256ull << 20)
int pm_muon_step_noalloc(const pm_matrix* mats, int n, const pm_hparams* hp,
                         const float* lr_dev, double lr_host, void* stream);

/* Workspace needed by pm_newton_schulz. */
size_t pm_ns_workspace_bytes(const pm_ns_matrix* mats, int n, const pm_hparams* hp);

/*
 * Newton–Schulz only: out_i = NS(in_i) in bf16, same shape as in_i.
 * Replaces torch.optim._muon._zeropower_via_newtonschulz, which PAN 2's
 * patch_muon swaps for _gram_newtonschulz_local (pan/optim/patch_muon.py:339).
 */
int pm_newton_schulz(const pm_ns_matrix* mats, int n, const pm_hparams* hp,
                     void* workspace, size_t workspace_bytes, void* stream);

/*
 * Fused Nesterov momentum over n contiguous elements. Replaces
 * muon_momentum_nesterov (pan/optim/muon_triton.py:54-108): buf is updated in
 * place and the update is written to `update` in update_dtype.
 */
int pm_momentum_nesterov(void* buf, int32_t buf_dtype,
                         const void* grad, int32_t grad_dtype,
                         void* update, int32_t update_dtype,
                         int64_t n, float momentum, int32_t nesterov, void* stream);

/*
 * Fused parameter step over n contiguous elements. Replaces step_param
 * (pan/optim/muon_triton.py:164-210): p <- p*(1 - lr*wd) - lr*adj_ratio*u,
 * fp32 math; lr from lr_dev when it is not NULL, else lr_host.
 */
int pm_step_param(void* param, int32_t param_dtype,
                  const void* update, int32_t update_dtype,
                  int64_t n, const float* lr_dev, double lr_host,
                  float weight_decay, double adj_ratio, void* stream);

/*
 * Symmetric gram C = X Xᵀ (bf16 in, fp32 accumulate, bf16 out) on the
 * upper-triangle tiles, mirrored. Replaces quack gemm_symmetric_out(X, X.mT)
 * (pan/optim/patch_muon.py:310). X is rows x cols with ld == cols, C is
 * rows x rows with ld == rows; rows and cols must be multiples of 256.
 * Needs pm_gram_workspace_bytes() of workspace.
 */
size_t pm_gram_workspace_bytes(void);
int pm_gram(const void* x, int64_t rows, int64_t cols, void* out,
            void* workspace, size_t workspace_bytes, void* stream);

/*
 * Symmetric product out = alpha * L Rᵀ + beta * D on m x m bf16 matrices
 * (fp32 accumulate, bf16 out). Only the upper triangle is computed (the
 * 256 x 256 tiles on and above the diagonal) and it is mirrored, so the
 * result is exactly symmetric. Replaces quack gemm_symmetric_out(L, R, out=out, C=D, alpha,
 * beta) and gemm_symmetric(L, R, C=D, beta=beta) as PAN 2's gram form calls
 * them (pan/optim/patch_muon.py:320-331), where R and D are symmetric (so
 * L Rᵀ = L R) and L, R commute. D may be NULL when beta == 0 (it is then not
 * read). All matrices have ld == m; m must be a multiple of 256. out must not
 * alias L, R or D.
 */
size_t pm_gemm_symmetric_workspace_bytes(void);
int pm_gemm_symmetric(const void* left, const void* right, const void* addend, void* out, int64_t m,
                      float alpha, float beta, void* workspace, size_t workspace_bytes, void* stream);

/*
 * The Adam / AdamW half of PAN 2's step (pan/optim/muon.py:155-164 builds
 * torch.optim.AdamW(fused=True) over the params Muon does not take). One
 * contiguous tensor and its state; the fields mirror the lists torch's fused
 * Adam receives (params, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs,
 * state_steps, torch/optim/adam.py:803-815).
 *   step: torch's state["step"], a float32 scalar on the device.
 *   max_exp_avg_sq: amsgrad only (NULL otherwise), dtype of exp_avg_sq.
 */
typedef struct pm_adam_tensor {
  void* param;
  void* grad; /* read; written (unscaled) only with a grad_scale */
  void* exp_avg;
  void* exp_avg_sq;
  void* max_exp_avg_sq;
  float* step;
  int64_t numel;
  int32_t param_dtype;
  int32_t grad_dtype;
  int32_t exp_avg_dtype;
  int32_t exp_avg_sq_dtype;
} pm_adam_tensor;

/* The scalars of torch's Adam param group (torch/optim/adam.py:88-101). */
typedef struct pm_adam_hparams {
  double beta1;
  double beta2;
  double eps;
  double weight_decay;
  int32_t amsgrad;
  int32_t maximize;
  int32_t decoupled_weight_decay; /* 1: AdamW (param *= 1 - lr*wd), 0: Adam (grad += wd*param) */
  int32_t reserved;
} pm_adam_hparams;

/*
 * One Adam / AdamW step over n tensors, in place. Replaces torch's
 * _fused_adam (torch/optim/adam.py:803-898): every step += 1, then per element
 * (fp32 arithmetic, each result rounded once to its storage dtype)
 *   p *= 1 - lr*wd (AdamW);  m = lerp(m, g, 1 - beta1);
 *   v = v*beta2 + (1 - beta2) g^2;  p += -(lr / (1 - beta1^step)) * m / (sqrt(v) / sqrt(1 - beta2^step) + eps)
 * (torch/optim/adam.py:414-547). lr from lr_dev (device float) when it is not
 * NULL, else lr_host. grad_scale (device float, or NULL) divides the grads,
 * which are written back unscaled, as torch's fused kernel leaves them;
 * found_inf (device float, or NULL) skips the update and the step count when
 * nonzero, as torch's fused path does for a GradScaler.
 * Needs pm_adam_workspace_bytes(n) of device workspace (the descriptor table).
 */
size_t pm_adam_workspace_bytes(int n);
int pm_adam_step(const pm_adam_tensor* tensors, int n, const pm_adam_hparams* hp, const float* lr_dev,
                 double lr_host, const float* grad_scale, const float* found_inf, void* workspace,
                 size_t workspace_bytes, void* stream);

/*
 * Opt-in launch timing (no counterpart in the reference, which has no
 * instrumentation; used by bench.py for live roofline figures). While enabled,
 * every launch of pm_muon_step / pm_newton_schulz records a HIP event on the
 * call's stream; pm_timing_read waits for those events and returns one record
 * per launch with its algorithmic work.
 */
enum pm_kernel_kind {
  PM_K_PROLOGUE = 0,  /* momentum + bf16 X + Σx² partials */
  PM_K_NORM = 1,      /* per-matrix 1/‖X‖ */
  PM_K_GRAM = 2,      /* A = X Xᵀ (symmetric) */
  PM_K_POLY = 3,      /* symmetric product: B = b A + c A² (standard form);
                         Z, Q, RZ and R updates (gram form) */
  PM_K_UPDATE = 4,    /* X <- a X + B X (gram form: X <- Q X at the reset) */
  PM_K_FINAL = 5,     /* last update fused with the parameter step */
  PM_K_QINIT = 6,     /* gram form: Q = Z + a I */
  PM_K_SMALL_CORE = 7, /* matrices with min(rows, cols) <= 128: gram and the
                         M x M part of one iteration (standard form) or of one
                         segment (gram form), in one launch */
  PM_K_ADAM = 8,       /* pm_adam_step: step counts and the element update */
  PM_K_REDUCE = 9      /* a K-split stage's second launch: the chunks' fp32
                         partial tiles summed in chunk order, then the stage's
                         epilogue (matrices of 512 <= Mp whose own tiles leave
                         most of the chip idle; flops 0, counted by the stage) */
};

typedef struct pm_launch_time {
  int32_t kind;        /* pm_kernel_kind */
  int32_t group;       /* workspace group within the call */
  int32_t iteration;   /* Newton–Schulz iteration (-1 for prologue/norm) */
  int32_t n_matrices;  /* matrices walked by this launch */
  double flops;        /* algorithmic FLOPs (GEMM launches) */
  double bytes;        /* algorithmic HBM bytes (prologue) */
  float ms;            /* event-measured duration */
  float reserved;
} pm_launch_time;

int pm_timing_enable(int on);
/* Returns the number of records written (<= max) and clears them; < 0 on error. */
int pm_timing_read(pm_launch_time* out, int max);

#ifdef __cplusplus
}
#endif

#endif /* PANMUON_H */
