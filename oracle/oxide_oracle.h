/*
 * oxide_oracle.h -- CPU restatement of oxide-torch's CPU path for the tensor hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP kernels in
 * liboxide_hip.so.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it.  The product never links, calls or falls back to it.
 *
 * Every function restates one piece of the reference's CPU evaluation or autograd, in the same
 * evaluation order and fp32 rounding sequence, and cites the reference file:line it follows
 * (paths relative to the tuna2134/oxide-beta checkout).  Build flags: -O2 -ffp-contract=off, no
 * fast-math, single-threaded.
 *
 * Pinning (what checks each function, all in tests/test_oracle_*.py):
 *   elementwise fwd/bwd, chain, plan   reference KATs tensor/mod.rs:568-574, jit.rs:721-736,
 *                                      exact numpy closed forms
 *   batch norm fwd/running/bwd         KATs nn.rs:761-790, jit.rs:763-782, finite difference
 *                                      tensor/mod.rs:627-686; torch fp64 batch_norm + autograd
 *   cross entropy fwd/bwd              KAT tensor/mod.rs:616-625 (exact); torch fp64
 *                                      cross_entropy + autograd; zero-logit closed form
 *   powi                               exact powers of two, integer powers vs fp64
 *   adamw                              torch.optim.AdamW in fp64; t=1 sign(g) closed form;
 *                                      optim.rs:168-208 loss-decrease property
 *   argmax (last index wins ties)      hand cases incl. ties, -0/+0 and NaN ordering
 *   conv2d fwd/bwd, avg_pool2d fwd/bwd KAT tensor/mod.rs:586-614 (exact); torch fp64 conv2d /
 *                                      avg_pool2d + autograd, grouped and strided cases
 *   initialized_weights                parity unpinned beyond range/determinism properties
 */
#ifndef OXIDE_ORACLE_H
#define OXIDE_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes shared with the tests (mirrors the reference's Error variants that this path
 * can raise: crates/oxide-torch/src/error.rs:1-56). */
#define ORO_OK 0
#define ORO_INVALID_SHAPE 1 /* Error::InvalidShape */
#define ORO_EXECUTION 2     /* Error::Execution */

/* ---- elementwise (evaluation.rs:21-34,638-640; jit.rs:503-517) ---- */
void oro_add(const float *a, const float *b, float *out, uint64_t n);
void oro_mul(const float *a, const float *b, float *out, uint64_t n);
void oro_relu(const float *x, float *out, uint64_t n);
/* autograd.rs:123-147 */
void oro_mul_backward(const float *grad, const float *other, float *out, uint64_t n);
void oro_relu_backward(const float *grad, const float *input, float *out, uint64_t n);
/* autograd.rs:94-108: current += incoming */
void oro_accumulate(float *current, const float *incoming, uint64_t n);
/* Plan executor for relu((a+b)*c) (jit.rs:479-560): three ops, three workspaces. */
void oro_chain_forward(const float *a, const float *b, const float *c, float *y, uint64_t n);
/* Backward of relu((a+b)*c) with upstream ones, via the reference VJPs in graph order
 * (autograd.rs:111-147). */
void oro_chain_backward_ones(const float *a, const float *b, const float *c, float *da, float *db,
                             float *dc, uint64_t n);

/* ---- batch norm 2d (NCHW) ---- */
/* evaluation.rs:490-535: mean, inverse std (epsilon added before sqrt). */
int oro_bn_batch_statistics(const float *x, uint64_t batch, uint64_t channels, uint64_t spatial,
                            float epsilon, float *mean, float *inv_std);
/* evaluation.rs:537-558: recomputes stats with epsilon 0, powi(-2), unbiased correction. */
int oro_bn_update_running(const float *x, uint64_t batch, uint64_t channels, uint64_t spatial,
                          float momentum, float *running_mean, float *running_var);
/* evaluation.rs:560-575 */
void oro_bn_running_statistics(const float *running_var, uint64_t channels, float epsilon,
                               float *inv_std);
/* evaluation.rs:577-597 */
void oro_bn_apply(const float *x, uint64_t batch, uint64_t channels, uint64_t spatial,
                  const float *weight, const float *bias, const float *mean, const float *inv_std,
                  float *y);
/* evaluation.rs:448-488: full forward (train: stats + running update + apply; eval: running). */
int oro_bn_forward(const float *x, uint64_t batch, uint64_t channels, uint64_t spatial,
                   const float *weight, const float *bias, float *running_mean, float *running_var,
                   int training, float momentum, float epsilon, float *y, float *saved_mean,
                   float *saved_inv_std);
/* autograd.rs:315-383: dx, dweight, dbias from saved statistics. */
void oro_bn_backward(const float *grad, const float *x, uint64_t batch, uint64_t channels,
                     uint64_t spatial, const float *weight, const float *mean,
                     const float *inv_std, int training, float *dx, float *dweight, float *dbias);

/* ---- cross entropy ---- */
/* evaluation.rs:622-636 */
int oro_class_index(float value, uint64_t classes, uint64_t *index);
/* evaluation.rs:599-620: mean NLL of row log-softmax. */
int oro_ce_forward(const float *logits, const float *targets, uint64_t batch, uint64_t classes,
                   float *loss);
/* autograd.rs:529-554: grad = (outer/B) * (softmax - onehot). */
int oro_ce_backward(const float *logits, const float *targets, uint64_t batch, uint64_t classes,
                    float outer_gradient, float *grad);

/* ---- AdamW (optim.rs:78-127) ---- */
/* compiler-rt __powisf2 algorithm, which Rust's f32::powi(i32) lowers to. */
float oro_powi(float a, int32_t b);
/* One update of one parameter tensor at optimizer step `step` (already incremented, as
 * optim.rs:140-152 does before visiting parameters). */
void oro_adamw_update(float *param, const float *grad, float *first_moment, float *second_moment,
                      uint64_t n, float learning_rate, float weight_decay, float beta1,
                      float beta2, float epsilon, int32_t step);

/* ---- conv2d / avg_pool2d (NCHW, OIHW weights) ---- */
/* evaluation.rs:334-397: out[n,oc,oy,ox] = bias[oc] + sum over (local channel, ky, kx). */
void oro_conv2d_forward(const float *input, const float *weight, const float *bias,
                        uint64_t batch, uint64_t in_channels, uint64_t height, uint64_t width,
                        uint64_t out_channels, uint64_t kernel_h, uint64_t kernel_w,
                        uint64_t stride, uint64_t padding, uint64_t groups, float *output);
/* autograd.rs:412-483: scatter-accumulated input, weight and bias gradients. */
void oro_conv2d_backward(const float *grad, const float *input, const float *weight,
                         uint64_t batch, uint64_t in_channels, uint64_t height, uint64_t width,
                         uint64_t out_channels, uint64_t kernel_h, uint64_t kernel_w,
                         uint64_t stride, uint64_t padding, uint64_t groups, float *dinput,
                         float *dweight, float *dbias);
/* evaluation.rs:399-445 */
void oro_avg_pool2d_forward(const float *input, uint64_t batch, uint64_t channels,
                            uint64_t height, uint64_t width, uint64_t kernel_h, uint64_t kernel_w,
                            uint64_t stride_h, uint64_t stride_w, float *output);
/* autograd.rs:485-527 */
void oro_avg_pool2d_backward(const float *grad, uint64_t batch, uint64_t channels,
                             uint64_t height, uint64_t width, uint64_t kernel_h,
                             uint64_t kernel_w, uint64_t stride_h, uint64_t stride_w,
                             float *dinput);

/* ---- models / driver helpers ---- */
/* nn.rs:657-674: deterministic variance-scaled init of an OIHW conv weight. */
void oro_initialized_weights(const uint64_t *shape, uint64_t input_channels_per_group,
                             float *out);
/* mnist_training.rs:201-218: argmax with total_cmp, last index wins ties. */
void oro_argmax_rows(const float *logits, uint64_t rows, uint64_t classes, uint64_t *out);

/* ---- MNIST data (crates/oxide-torch/src/data/mnist.rs) ---- */
/* mnist.rs:118-121: (f32::from(pixel) / 255.0 - 0.1307) / 0.3081 per byte. */
void oro_mnist_normalize(const uint8_t *pixels, uint64_t n, float *out);
/* mnist.rs:191-199: deterministic_shuffle of `values` in place. */
void oro_mnist_shuffle(uint64_t *values, uint64_t n);

#ifdef __cplusplus
}
#endif
#endif
