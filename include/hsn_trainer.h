/*
 * hsn_trainer.h -- the trainer's per-step passes after backward() on MI355X (gfx950): the AdamW
 * step of ordinary and of stacked unit tensors, the weight average's lerp, the float64 clip's
 * scaling, a copy and the update caps' two passes, each one launch over a list of fp32 tensors.
 *
 * Replaces the reference's hsn_tr_* kernels (kernels/cuda/hsn_trainer.cu:60-182), which its
 * python/hsn/kernels/trainer.py:111-229 launches through a private descriptor
 * (kernels/include/hsn_trainer_launch.h:13-27); here a host passes plain arrays instead: one
 * array of device pointers per operand ("row") and one of element counts, n tensors, any n (a long
 * list takes several launches). Each pass equals, bit for bit, the PyTorch multi-tensor
 * operations it replaces (python/hsn/train/lazy_adam.py:462-486,573-626; weight_ema, grad_norm,
 * update_limit). Tensors are contiguous fp32 on the stream's device; `stream` is a hipStream_t
 * (NULL: the default stream); functions return once the work is enqueued, with the status codes
 * of hsn_ops.h and the message in hsn_win_last_error().
 */
#ifndef HSN_TRAINER_H
#define HSN_TRAINER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * LazyAdamW._dense_steps (reference hsn_trainer.cu:60-90, trainer.py:111-144): for every element
 *   p *= coefs[0] (when weight_decay_on);  m = lerp(m, g, coefs[1]);  v *= coefs[2];
 *   v = addcmul(v, g, g, coefs[3]);  den = sqrt(v) * coefs[4] + coefs[5];
 *   p = addcdiv(p, m, den, coefs[6])
 * coefs: 1 - lr wd, 1 - beta1, beta2, 1 - beta2, 1 / sqrt(1 - beta2^t) (rounded from double, as
 * torch's division of a list by a scalar), eps, -lr / (1 - beta1^t). params, exp_avgs and
 * exp_avg_sqs in place.
 */
int hsn_tr_adamw(float* const* params, float* const* grads, float* const* exp_avgs,
                 float* const* exp_avg_sqs, const int64_t* numels, int n, int weight_decay_on,
                 const float* coefs, void* stream);

/*
 * LazyAdamW._unit_step for stacked unit tensors [n_units, ...] sharing their per-unit step
 * counts (reference hsn_trainer.cu:92-130, trainer.py:147-191): with unit u = element / (numel
 * / n_units) and unit_coefs [6][n_units] = (active 1 / 0, decay, lerp weight, the second moment's
 * factor, sqrt(1 - beta2^t), lr / (1 - beta1^t)), the inactive units' 1, 1, 0, 1, 1, 0:
 *   g = active ? grad : 0;  p *= decay (when weight_decay_on);  m = lerp(m, g, w);  v *= b2f;
 *   v = addcmul(v, g, g, one_minus_beta2);  den = sqrt(v) / bc2s + eps;
 *   p = addcdiv(p, m * step, den, -1).   n_units in [1, 64].
 */
int hsn_tr_adamw_units(float* const* params, float* const* grads, float* const* exp_avgs,
                       float* const* exp_avg_sqs, const int64_t* numels, int n, int n_units,
                       int weight_decay_on, const float* unit_coefs, float one_minus_beta2,
                       float eps, void* stream);

/* torch._foreach_lerp_(selfs, ends, weight) (reference hsn_trainer.cu:132-139, trainer.py:194). */
int hsn_tr_lerp(float* const* selfs, float* const* ends, const int64_t* numels, int n,
                float weight, void* stream);

/*
 * grad = f32(f64(grad) * coefficient), every gradient (the float64 clip; reference
 * hsn_trainer.cu:141-151, trainer.py:199-205); coefficient: one f64 on the device.
 */
int hsn_tr_scale64(float* const* grads, const int64_t* numels, int n, const double* coefficient,
                   void* stream);

/* dst = src (reference hsn_trainer.cu:153-158, trainer.py:208-210). */
int hsn_tr_copy(float* const* dsts, float* const* srcs, const int64_t* numels, int n,
                void* stream);

/*
 * UpdateLimiter.apply's first pass (reference hsn_trainer.cu:160-170, trainer.py:213-222):
 * old_squares = old^2, delta_squares = (param - old)^2.
 */
int hsn_tr_limit_squares(float* const* params, float* const* olds, float* const* old_squares,
                         float* const* delta_squares, const int64_t* numels, int n, void* stream);

/*
 * UpdateLimiter.apply's projection (reference hsn_trainer.cu:172-182, trainer.py:225-229):
 * groups[j] holds tensor j's group as two f32 on the device, [scale, clipped 1 / 0];
 * param = old + (param - old) * scale where clipped, then applied_squares = (param - old)^2.
 */
int hsn_tr_limit_project(float* const* params, float* const* olds, float* const* applied_squares,
                         float* const* groups, const int64_t* numels, int n, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HSN_TRAINER_H */
