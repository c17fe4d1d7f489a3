"""Writes kael with the optional MI355X device branches into oracle/_ref/fused/ (test build only).

TEST INFRASTRUCTURE: the reference's sources are read where they lie under /root/reference and
the patched copies are written only to oracle/_ref/fused/ (git-ignored); nothing here ships.
It applies the optional kael-side patches (one device branch per site), so that the tests can run kael's
training configs with kael's own host code calling the backend's fused entry points
(kael.cpp_amd/host/kd_kael_extensions.h):

  include/kael/device_kernels.h      + one include of kd_kael_extensions.h (the declarations)
  src/ops/nn.cpp                     the device interface include; device branches of softmax and
                                     log_softmax (reference :147-181), standardize (:244-271),
                                     cross_entropy_losses (:183-210) and
                                     detail::cross_entropy_gradient (:214-240)
  src/autograd/functions_math.cpp    GELU backward without the host round trip (:221-231)
  src/autograd/functions_reduce.cpp  SoftmaxBackward / LogSoftmaxBackward along the last dim
                                     (:150-164) and StandardizeBackward (:176-192) as one row
                                     kernel each
  src/autograd/functions_linalg.cpp  the gradient of a 2-D weight shared by every batch item of
                                     the left operand (kael's Linear) as one product over the
                                     folded batch, X^T . g with K = all tokens, instead of one
                                     product per batch item and a sum over the batch (:37-44)
  src/ops/linalg.cpp                 multiply_batches reads transposed / broadcast operands in
                                     place (:56-76)
  src/optim/optimizer.cpp            SGD (no momentum, :60-80) updates a contiguous device
                                     parameter in one kernel; Adam / AdamW (:93-120) collects the
                                     contiguous device parameters and updates them in one call
  src/ops/reduce.cpp                 prod (:362-369), argmax / argmin (:399-421) and all / any
                                     (:423-451) of a device tensor on the device instead of through
                                     a host copy (the same planning: plan_reduction's kept-first
                                     permutation, then one call over contiguous chunks); sum
                                     over the leading dims of a contiguous tensor (:316-319)
                                     read in place, without plan_reduction's transposed copy
  src/ops/sequence.cpp               cumsum (:95-117) of a device tensor on the device
  src/autograd/node.cpp              AccumulateGrad::apply (:18-36): a device gradient that nothing
                                     else references becomes the leaf's first gradient without the
                                     clone's device copy
  src/ops/indexing.cpp, inplace.cpp  gather (:143-156) and scatter_add_ (:160-178) with broadcast 1-D
                                     indices (index_select, index_add_): one range check of the
                                     line (kd_index_bounds) and the indices read in place, instead
                                     of a contiguous copy checked by two reductions and two reads
  src/ops/nn.cpp, src/nn/loss.cpp    the cross-entropy targets' range check (:97-98, :27-28) in one
                                     call
  src/random.cpp, src/nn/functional.cpp
                                     dropout (functional.cpp:32-39) of a contiguous f32 / f64 device
                                     tensor: the bernoulli mask drawn on the device from kael's
                                     generator (random.cpp:106-110), output and mask in one launch,
                                     the generator advanced as the host draws advance it
  src/nn/transformer.cpp             CausalSelfAttention::forward (:103-138) without a cache or
                                     dropout, f32 heads of 64: one device call forward and one node
                                     (one launch) backward (kd_causal_attention); with a cache and
                                     no gradient recorded, the new queries against the cached keys
                                     and values read in place, one device call
                                     (kd_cached_attention);
                                     nn::generate (:256-295) with temperature 0, the KV cache and a
                                     batch-1 prompt on the device runs on the decode engine
                                     (kd_gpt_*), token for token the greedy sequence of the loop

Each edit is anchored on a line of the reference file that must occur exactly once; a missing
or repeated anchor is an error, so a changed reference fails loudly instead of building
something else. The inserted code is this repository's own.

Usage: python oracle/kael_fused.py REF_DIR OUT_DIR
"""
from __future__ import annotations

import sys
from pathlib import Path

SOFTMAX_BRANCH = """        if (x.device() != Device::CPU && x.dim() > 0 && x.is_contiguous() &&
            dim_position(dim, x.dim()) == static_cast<std::size_t>(x.dim() - 1)) {
            // MI355X: one fused row kernel instead of max, sub, exp, sum and div launches.
            Tensor out = empty(x.shape(), x.dtype(), x.device());
            device::softmax_rows(x.dtype(), out.device_data(), x.device_data(), x.numel() / x.size(-1),
                                 x.size(-1), %s);
            return out;
        }
"""

STANDARDIZE_BRANCH = """        if (x.device() != Device::CPU) {
            // MI355X: one fused row kernel (mean and population variance in double).
            const std::int64_t row_size =
                numel(Shape(x.shape().end() - static_cast<std::ptrdiff_t>(normalized_dims), x.shape().end()));
            Tensor out = empty(x.shape(), x.dtype(), x.device());
            device::standardize_rows(x.dtype(), out.device_data(), x.device_data(), x.numel() / row_size, row_size,
                                     eps);
            return out;
        }
"""

CROSS_ENTROPY_BRANCH = """    if (logits.device() != Device::CPU) {
        // MI355X: per-row losses in one kernel; the backward is detail::cross_entropy_gradient.
        Tensor out = autograd::without_grad([&] {
            const Tensor x = as_floating(logits).contiguous();
            const Tensor classes = targets.contiguous();
            Tensor losses = empty({x.size(0)}, x.dtype(), x.device());
            if (x.numel() > 0) {
                device::cross_entropy_rows(x.dtype(), losses.device_data(), x.device_data(),
                                           reinterpret_cast<const std::int64_t*>(classes.device_data()),
                                           x.size(0), x.size(1));
            }
            return losses;
        });
        autograd::record_cross_entropy(out, logits, targets);
        return out;
    }
"""

CROSS_ENTROPY_GRAD_BRANCH = """    if (x.device() != Device::CPU) {
        // MI355X: softmax(x) * w[row] - w[row] * onehot(target) in one kernel.
        Tensor out = empty(x.shape(), x.dtype(), x.device());
        if (x.numel() > 0) {
            device::cross_entropy_grad(x.dtype(), out.device_data(), x.device_data(),
                                       reinterpret_cast<const std::int64_t*>(classes.device_data()),
                                       weights.to(x.dtype()).contiguous().device_data(), x.size(0), x.size(1));
        }
        return out;
    }
"""

GELU_BACKWARD_BRANCH = """                          if (saved.get().device() != Device::CPU) {
                              // MI355X: g * gelu'(x) as one element kernel, no host round trip.
                              const NoGradGuard guard;
                              const Tensor xs = saved.get();
                              const DType dtype = is_floating_point(xs.dtype()) ? xs.dtype() : DType::F32;
                              TensorIterator iterator;
                              iterator.allocate_output(dtype).add_input(xs.to(dtype)).add_input(g.to(dtype)).build();
                              device::elementwise(device::gelu_backward_op(approximate), dtype, dtype,
                                                  iterator.device_layout(), {});
                              return iterator.output();
                          }
"""

STRIDES_HELPER = """// MI355X: the element stride of dims [lo, hi) of an expanded operand when they flatten to one
// (contiguous or broadcast dims; size-1 dims skipped, 0 when all have size 1); false otherwise.
bool flat_group_stride(const Tensor& v, std::int64_t lo, std::int64_t hi, std::int64_t& stride) {
    stride = 0;
    bool first = true;
    std::int64_t span = 0;
    for (std::int64_t i = hi - 1; i >= lo; --i) {
        if (v.size(i) == 1) {
            continue;
        }
        if (first) {
            stride = v.stride(i);
            span = v.stride(i) * v.size(i);
            first = false;
        } else if (v.stride(i) == span) {
            span *= v.size(i);
        } else {
            return false;
        }
    }
    return true;
}

// MI355X: element strides {batch, row, column} of an expanded operand whose batch dims flatten
// to one stride; false when they do not.
bool flat_batch_strides(const Tensor& v, std::int64_t* strides) {
    const std::int64_t d = v.dim();
    strides[1] = v.stride(d - 2);
    strides[2] = v.stride(d - 1);
    return flat_group_stride(v, 0, d - 2, strides[0]);
}

"""

MATMUL_BRANCH = """    if (a.device() != Device::CPU && is_floating_point(dtype)) {
        // MI355X: transposed and batch-broadcast operands read in place (no expand/reshape copies).
        const Tensor va = a.to(dtype).expand(with_matrix_dims(batch, rows, inner));
        const Tensor vb = b.to(dtype).expand(with_matrix_dims(batch, inner, columns));
        std::int64_t sa[3];
        std::int64_t sb[3];
        if (flat_batch_strides(va, sa) && flat_batch_strides(vb, sb)) {
            Tensor out = empty(with_matrix_dims(batch, rows, columns), dtype, a.device());
            const std::int64_t so[3] = {rows * columns, columns, 1};
            device::matmul_strided(dtype, va.device_data(), vb.device_data(), out.device_data(),
                                   {numel(batch), rows, inner, columns}, sa, sb, so);
            return out;
        }
        // Batch dims that flatten in two groups, [0, cut) and [cut, end) (attention's per-head
        // views: [batch, head] over a [batch, token, head, dim] tensor): one product over both.
        const std::int64_t batch_dims = va.dim() - 2;
        for (std::int64_t cut = 1; cut < batch_dims; ++cut) {
            std::int64_t heads = 1;
            for (std::int64_t i = cut; i < batch_dims; ++i) {
                heads *= va.size(i);
            }
            std::int64_t head_strides[3];
            if (heads < 1 || !flat_group_stride(va, 0, cut, sa[0]) || !flat_group_stride(va, cut, batch_dims, head_strides[0]) ||
                !flat_group_stride(vb, 0, cut, sb[0]) || !flat_group_stride(vb, cut, batch_dims, head_strides[1])) {
                continue;
            }
            sa[1] = va.stride(-2);
            sa[2] = va.stride(-1);
            sb[1] = vb.stride(-2);
            sb[2] = vb.stride(-1);
            head_strides[2] = rows * columns;
            Tensor out = empty(with_matrix_dims(batch, rows, columns), dtype, a.device());
            const std::int64_t so[3] = {heads * rows * columns, columns, 1};
            device::matmul_strided_heads(dtype, va.device_data(), vb.device_data(), out.device_data(),
                                         {numel(batch), rows, inner, columns}, sa, sb, so, heads, head_strides);
            return out;
        }
    }
"""

ADAM_PENDING = """    // MI355X: the updates of device parameters are collected and run as one device call over the
    // list (a launch per 32 tensors instead of one per tensor). The list is flushed before
    // anything that must see its updates: a parameter on kael's composed path, a change of dtype,
    // or a tensor sharing storage with one already listed; so the results are those of the
    // sequential loop.
    std::vector<device::AdamTensor> pending;
    std::unordered_set<const void*> pending_storages;
    DType pending_dtype = DType::F32;
    const bool decoupled = options_.weight_decay > 0.0 && mode_ == WeightDecayMode::Decoupled;
    const auto flush = [&] {
        if (!pending.empty()) {
            device::adam_step_many(pending_dtype, pending, learning_rate(), options_.beta1, options_.beta2,
                                   options_.epsilon, options_.weight_decay, decoupled);
        }
        pending.clear();
        pending_storages.clear();
    };
"""

ADAM_BRANCH = """        if (parameter.device() != Device::CPU && is_floating_point(parameter.dtype()) &&
            parameter.is_contiguous() && stored->dtype() == parameter.dtype() && stored->is_contiguous() &&
            first_moments_[i].is_contiguous() && second_moments_[i].is_contiguous()) {
            const void* storages[4] = {parameter.impl()->storage.get(), stored->impl()->storage.get(),
                                       first_moments_[i].impl()->storage.get(),
                                       second_moments_[i].impl()->storage.get()};
            bool flush_first = !pending.empty() && parameter.dtype() != pending_dtype;
            for (const void* storage : storages) {
                flush_first = flush_first || pending_storages.count(storage) != 0;
            }
            if (flush_first) {
                flush();
            }
            pending_dtype = parameter.dtype();
            pending.push_back({parameter.device_data(), stored->device_data(), first_moments_[i].device_data(),
                               second_moments_[i].device_data(), parameter.numel(), steps_[i]});
            pending_storages.insert(std::begin(storages), std::end(storages));
            // The in-place ops below bump each storage's version once per op.
            parameter.impl()->storage->bump_version();
            if (decoupled) {
                parameter.impl()->storage->bump_version();
            }
            for (int bump = 0; bump < 2; ++bump) {
                first_moments_[i].impl()->storage->bump_version();
                second_moments_[i].impl()->storage->bump_version();
            }
            continue;
        }
        flush();
"""

SGD_BRANCH = """        if (options_.momentum == 0.0 && parameter.device() != Device::CPU &&
            is_floating_point(parameter.dtype()) && parameter.is_contiguous() &&
            stored->dtype() == parameter.dtype() && stored->is_contiguous()) {
            // MI355X: parameter.sub_((g + p * weight_decay) * lr) in one kernel.
            device::sgd_step(parameter.dtype(), parameter.device_data(), stored->device_data(), parameter.numel(),
                             learning_rate(), options_.weight_decay);
            parameter.impl()->storage->bump_version();
            continue;
        }
"""

WEIGHT_GRADIENT_BRANCH = """                     if (g.device() != Device::CPU && !layout.left_is_vector && !layout.right_is_vector &&
                         shape.size() == 2 && left.get().dim() > 2 && left.get().size(-1) > 0 &&
                         g.size(-1) > 0) {
                         // MI355X: the weight is shared by every batch item, so its gradient is one
                         // product over the folded batch (K = every row of every item). An empty
                         // last dim keeps kael's per-item path (the fold would divide by zero).
                         // Computed as (g^T . X)^T: the product lands in the layout of the weight
                         // behind the transposed view (Linear's weight.T()), so that view's backward
                         // hands the weight a contiguous gradient and no transposing copy is made.
                         const Tensor x = left.get();
                         const Tensor flat_x = x.reshape({x.numel() / x.size(-1), x.size(-1)});
                         const Tensor flat_g = g.reshape({g.numel() / g.size(-1), g.size(-1)});
                         return matmul(flat_g.mT(), flat_x).mT().to(dtype);
                     }
"""

LINEAR_BRANCH = """    if (bias_ && input.device() != Device::CPU && input.dim() >= 2 && is_floating_point(input.dtype()) &&
        input.is_contiguous() && weight_.dim() == 2 && weight_.is_contiguous() && input.size(-1) == weight_.size(1) &&
        weight_.dtype() == input.dtype() && bias_->dtype() == input.dtype() && bias_->is_contiguous() &&
        weight_.device() == input.device() && bias_->device() == input.device()) {
        // MI355X: matmul(input, weight.T()) + bias with the add as the product's epilogue, over the
        // same batched operands as the matmul device branch (so the same kernel and the same
        // product bits), one launch instead of two. The graph is the composed one: a stand-in for
        // the product (MatmulBackward and AddBackward read neither the product nor the sum).
        const Tensor weight_t = weight_.T();
        const std::int64_t inner = input.size(-1);
        const std::int64_t rows = input.size(-2);
        const std::int64_t columns = weight_.size(0);
        Shape shape(input.shape().begin(), input.shape().end() - 1);
        shape.push_back(columns);
        const std::int64_t batches = input.numel() / std::max<std::int64_t>(1, rows * inner);
        Tensor out = empty(shape, input.dtype(), input.device());
        const std::int64_t sa[3] = {rows * inner, inner, 1};
        const std::int64_t sb[3] = {0, 1, inner};
        const std::int64_t so[3] = {rows * columns, columns, 1};
        device::matmul_strided_bias(input.dtype(), input.device_data(), weight_t.device_data(), out.device_data(),
                                    {batches, rows, inner, columns}, sa, sb, so, bias_->device_data());
        if (autograd::should_record(out, {&input, &weight_t, &*bias_})) {
            const Tensor product = out.detach();
            autograd::record_matmul(product, input, weight_t);
            autograd::record_add(out, product, *bias_);
        }
        return out;
    }
"""

LAYER_NORM_BRANCH = """    if (input.device() != Device::CPU && input.numel() > 0 && is_floating_point(input.dtype()) &&
        weight_.dtype() == input.dtype() && bias_.dtype() == input.dtype() && weight_.device() == input.device() &&
        bias_.device() == input.device() && weight_.is_contiguous() && bias_.is_contiguous()) {
        // MI355X: standardize, * weight and + bias in one launch that also keeps the standardized
        // rows; one node for the backward of all three (grad_in, and the weight and bias column
        // sums, in two launches), computed once for the node's three inputs.
        const std::int64_t cols = numel(normalized_shape_);
        const std::int64_t rows = input.numel() / cols;
        const DType dtype = input.dtype();
        const Tensor x = autograd::without_grad([&] { return input.contiguous(); });
        const Tensor standardized = empty(input.shape(), dtype, input.device());
        Tensor out = empty(input.shape(), dtype, input.device());
        device::layer_norm_rows(dtype, out.device_data(), standardized.device_data(), x.device_data(), rows, cols, eps_,
                                weight_.device_data(), bias_.device_data());
        if (autograd::should_record(out, {&input, &weight_, &bias_})) {
            struct Gradients {
                std::optional<Tensor> input, weight, bias;
                int pending = 0;  // node inputs that still have to take their gradient
                int needed = 0;
            };
            auto state = std::make_shared<Gradients>();
            state->needed = int{input.requires_grad()} + int{weight_.requires_grad()} + int{bias_.requires_grad()};
            auto take = [state, saved_x = autograd::SavedTensor(x), saved_y = autograd::SavedTensor(standardized),
                         saved_w = autograd::SavedTensor(weight_), rows, cols, dtype, eps = eps_,
                         shape = input.shape(), parameter_shape = weight_.shape()](const Tensor& g, int which) {
                if (state->pending == 0) {
                    const Tensor gc = g.contiguous();
                    Tensor grad_in = empty(shape, dtype, g.device());
                    Tensor grad_w = empty(parameter_shape, dtype, g.device());
                    Tensor grad_b = empty(parameter_shape, dtype, g.device());
                    device::layer_norm_rows_backward(dtype, grad_in.device_data(), grad_w.device_data(),
                                                     grad_b.device_data(), saved_x.get().device_data(),
                                                     saved_y.get().device_data(), gc.device_data(),
                                                     saved_w.get().device_data(), rows, cols, eps);
                    state->input = std::move(grad_in);
                    state->weight = std::move(grad_w);
                    state->bias = std::move(grad_b);
                    state->pending = state->needed;
                }
                std::optional<Tensor>& slot = which == 0 ? state->input : which == 1 ? state->weight : state->bias;
                Tensor result = std::move(*slot);
                slot.reset();
                --state->pending;
                return result;
            };
            autograd::set_history(out, "LayerNormBackward", {input, weight_, bias_},
                                  {[take](const Tensor& g) { return take(g, 0); },
                                   [take](const Tensor& g) { return take(g, 1); },
                                   [take](const Tensor& g) { return take(g, 2); }});
        }
        return out;
    }
"""

MASKED_FILL_BRANCH = """    if (t.device() != Device::CPU && mask.dtype() == DType::Bool &&
        broadcast_shapes(t.shape(), mask.shape()) == t.shape()) {
        // MI355X: one pass out = mask ? value : t into a fresh tensor, instead of a clone of t that
        // masked_fill_ then rewrites (the same element function and operands as masked_fill_).
        Tensor out = autograd::without_grad([&] {
            Tensor filled = empty(t.shape(), t.dtype(), t.device());
            TensorIterator iterator;
            iterator.add_output(filled).add_input(t).add_input(mask.to(t.dtype())).build();
            dispatch(t.dtype(), [&]<typename T>() {
                functions::MaskedFill<T> fill{value.as<T>()};
                detail::run_typed<T, T, 2>(iterator, fill);
            });
            return filled;
        });
        autograd::record_masked_fill(out, t, mask);
        return out;
    }
"""

ACCUMULATE_BRANCH = """    // MI355X: a device gradient that nothing else references (the engine's buffer holds its only
    // handle, and it spans its whole storage contiguously) becomes the leaf's first gradient as
    // is, instead of through clone(), which would copy it: the values are the clone's and nothing
    // else can observe the difference.
    if (gradient.device() != Device::CPU && leaf_->autograd && !leaf_->autograd->grad &&
        gradient.impl().use_count() == 1 && gradient.impl()->storage.use_count() == 1 &&
        !gradient.impl()->autograd && gradient.is_contiguous() && gradient.impl()->offset == 0 &&
        gradient.nbytes() == gradient.impl()->storage->nbytes()) {
        leaf_->autograd->grad = gradient;
        return {};
    }
"""

LEFT_WEIGHT_GRADIENT_BRANCH = """                     if (g.device() != Device::CPU && !layout.left_is_vector && !layout.right_is_vector &&
                         shape.size() == 2 && right.get().dim() > 2 && g.size(-1) > 0 && g.size(-2) > 0 &&
                         right.get().size(-2) > 0) {
                         // MI355X: a 2-D left operand shared by every batch item (kael's tied LM head,
                         // weight . h^T): its gradient is one product over the folded batch,
                         // (g^T)_flat^T . (right^T)_flat with K = every batch item's columns, instead
                         // of one product per item and a sum over the batch. The reshapes are views
                         // when the batch and column dims flatten (the head's gradient is a
                         // transposed view of a contiguous tensor, so they do).
                         const Tensor gt = g.transpose(-2, -1);
                         const Tensor rt = right.get().transpose(-2, -1);
                         const Tensor flat_g = gt.reshape({gt.numel() / gt.size(-1), gt.size(-1)});
                         const Tensor flat_r = rt.reshape({rt.numel() / rt.size(-1), rt.size(-1)});
                         return matmul(flat_g.mT(), flat_r).to(dtype);
                     }
"""

LEADING_REDUCE_HELPER = """// MI355X: a contiguous tensor reduced over its leading dims (an [outer, inner] matrix reduced
// over its rows: bias and LayerNorm gradients summed over every token) as one
// device::reduce_columns call that reads it in place; nullopt for any other case, which keeps
// plan_reduction's transposed copy.
std::optional<Tensor> device_leading_reduce(const Tensor& t, const Dims& dims, bool keepdim, device::ReduceOp op,
                                            DType dtype) {
    if (t.dim() < 2 || !t.is_contiguous() || t.numel() == 0) {
        return std::nullopt;
    }
    const std::vector<bool> reduced = reduced_positions(t, dims);
    std::size_t lead = 0;
    while (lead < reduced.size() && reduced[lead]) {
        ++lead;
    }
    if (lead == 0 || lead == reduced.size()) {
        return std::nullopt;
    }
    for (std::size_t i = lead; i < reduced.size(); ++i) {
        if (reduced[i]) {
            return std::nullopt;
        }
    }
    Shape output_shape;
    std::int64_t outer = 1;
    std::int64_t inner = 1;
    for (std::size_t i = 0; i < reduced.size(); ++i) {
        if (i < lead) {
            outer *= t.shape()[i];
            if (keepdim) {
                output_shape.push_back(1);
            }
        } else {
            inner *= t.shape()[i];
            output_shape.push_back(t.shape()[i]);
        }
    }
    Tensor out = empty(output_shape, dtype, t.device());
    device::reduce_columns(op, dtype, t.dtype(), out.device_data(), t.device_data(), outer, inner);
    return out;
}

"""

LEADING_SUM_BRANCH = """    if (std::optional<Tensor> columns = device_leading_reduce(
            t, dims, keepdim, device::ReduceOp::Sum, is_floating_point(t.dtype()) ? t.dtype() : DType::I64)) {
        return *columns;
    }
"""

REDUCE_HELPERS = """// MI355X: the reductions below run on the device over the same plan as device_reduce.
Tensor device_prod(const Tensor& t, const Dims& dims, bool keepdim) {
    const Reduction reduction = plan_reduction(t, dims, keepdim);
    Tensor out = empty(reduction.output_shape, is_floating_point(t.dtype()) ? t.dtype() : DType::I64, t.device());
    device::reduce_extra(device::ExtraReduceOp::Prod, reduction.data.dtype(), out.device_data(),
                         reduction.data.device_data(), reduction.chunk_size, reduction.output_count);
    return out;
}

Tensor device_logical(const Tensor& t, const Dims& dims, bool keepdim, device::ExtraReduceOp op) {
    const Reduction reduction = plan_reduction(t, dims, keepdim);
    Tensor out = empty(reduction.output_shape, DType::Bool, t.device());
    device::reduce_extra(op, reduction.data.dtype(), out.device_data(), reduction.data.device_data(),
                         reduction.chunk_size, reduction.output_count);
    return out;
}

Tensor device_arg_extreme(const Tensor& t, const Dims& dims, bool keepdim, bool largest, const char* op) {
    const Reduction reduction = plan_nonempty_reduction(t, dims, keepdim, op);
    Tensor out = empty(reduction.output_shape, DType::I64, t.device());
    device::arg_reduce(largest, reduction.data.dtype(), reinterpret_cast<std::int64_t*>(out.device_data()),
                       reduction.data.device_data(), reduction.chunk_size, reduction.output_count);
    return out;
}

"""

PROD_BRANCH = """    if (on_device(t)) {
        Tensor out = device_prod(t, dims, keepdim);
        autograd::record_prod(out, t, dims, keepdim);
        return out;
    }
"""

LOGICAL_BRANCH = """    if (on_device(t)) {
        return device_logical(t, dims, keepdim, device::ExtraReduceOp::%s);
    }
"""

ARG_BRANCH = """    if (on_device(t)) {
        return device_arg_extreme(%s, %s, %s);
    }
"""

CUMSUM_BRANCH = """    if (t.device() != Device::CPU) {
        // MI355X: running sums on the device instead of through a host copy.
        Tensor out = autograd::without_grad([&] {
            const Tensor rows = t.detach().transpose(dim, -1).to(dtype).contiguous();
            Tensor totals = empty(rows.shape(), dtype, rows.device());
            if (rows.numel() > 0) {
                device::cumsum_rows(dtype, totals.device_data(), rows.device_data(), rows.size(-1),
                                    rows.numel() / rows.size(-1));
            }
            return totals.transpose(dim, -1).contiguous();
        });
        autograd::record_cumsum(out, t, dim);
        return out;
    }
"""

ROW_BACKWARD_HELPERS = """// MI355X: the backward passes of softmax / log_softmax along the last dim and of standardize as
// one row kernel each; no value when the operands do not fit (kael's composed path runs then).
std::optional<Tensor> fused_softmax_backward(const Tensor& y, const Tensor& g, std::int64_t dim, bool log) {
    if (y.device() == Device::CPU || !is_floating_point(y.dtype()) || g.dtype() != y.dtype() || y.dim() == 0 ||
        y.numel() == 0 || g.shape() != y.shape() || wrap_dim(dim, y.dim()) != y.dim() - 1) {
        return std::nullopt;
    }
    const Tensor ys = y.contiguous();
    const Tensor gs = g.contiguous();
    Tensor out = empty(y.shape(), y.dtype(), y.device());
    device::softmax_rows_backward(y.dtype(), out.device_data(), ys.device_data(), gs.device_data(),
                                  y.numel() / y.size(-1), y.size(-1), log);
    return out;
}

std::optional<Tensor> fused_standardize_backward(const Tensor& x, const Tensor& y, const Tensor& g,
                                                 std::int64_t normalized_dims, double eps) {
    if (y.device() == Device::CPU || !is_floating_point(y.dtype()) || x.dtype() != y.dtype() ||
        g.dtype() != y.dtype() || y.numel() == 0 || x.shape() != y.shape() || g.shape() != y.shape()) {
        return std::nullopt;
    }
    std::int64_t row_size = 1;
    for (std::int64_t i = 1; i <= normalized_dims; ++i) {
        row_size *= y.size(-i);
    }
    const Tensor xs = x.contiguous();
    const Tensor ys = y.contiguous();
    const Tensor gs = g.contiguous();
    Tensor out = empty(y.shape(), y.dtype(), y.device());
    device::standardize_rows_backward(y.dtype(), out.device_data(), xs.device_data(), ys.device_data(),
                                      gs.device_data(), y.numel() / row_size, row_size, eps);
    return out;
}

"""

SOFTMAX_BACKWARD_BRANCH = """                        if (auto fused = fused_softmax_backward(y.get(), g, dim, %s)) {
                            return *fused;
                        }
"""

STANDARDIZE_BACKWARD_BRANCH = """                if (auto fused = fused_standardize_backward(saved.get(), y.get(), g, normalized_dims, eps)) {
                    return *fused;
                }
"""

GENERATE_HELPER = """// MI355X: generation with a KV cache of a batch-1 prompt on the device runs on the backend's
// decode engine (one captured step per token, the greedy pick or sample_next on the device) when
// the engine takes the model's shape and the temperature (0, or a positive finite float); no
// value otherwise, and the loop of generate() runs.
std::optional<Tensor> device_generate(GPT& model, const Tensor& prompt, const GenerateOptions& options) {
    const GptConfig& config = model.config();
    const bool sampled = options.temperature != 0.0;
    const float temperature = static_cast<float>(options.temperature);
    if (prompt.device() == Device::CPU || !options.use_cache || prompt.size(0) != 1 || options.max_new_tokens == 0 ||
        config.dtype != DType::F32 || prompt.dtype() != DType::I64 ||
        (sampled && (!(temperature > 0.0f) || !std::isfinite(temperature) ||
                     config.vocab_size > device::kGptSampleMaxVocab))) {
        return std::nullopt;
    }
    const device::GptEngineShape shape{config.vocab_size, config.max_positions, config.layers,
                                       config.heads,      config.dimension,     config.tanh_gelu};
    if (!device::gpt_engine_supported(shape)) {
        return std::nullopt;
    }
    const std::vector<NamedTensor> named = model.named_parameters();
    for (const auto& entry : named) {
        const Tensor& p = entry.second;
        if (p.device() != prompt.device() || p.dtype() != DType::F32 || !p.is_contiguous()) {
            return std::nullopt;
        }
    }
    struct Engine {
        void* handle;
        ~Engine() { device::gpt_engine_destroy(handle); }
    } engine{device::gpt_engine_create(shape)};
    for (const auto& entry : named) {
        device::gpt_engine_load(engine.handle, entry.first.c_str(), entry.second.device_data(), entry.second.numel());
    }
    const Tensor host_prompt = prompt.cpu().contiguous();
    const std::int64_t length = host_prompt.size(1);
    const std::int64_t* ids = host_prompt.data_ptr<std::int64_t>();
    // Sampled picks take kael's generator's next draws in order (one per token, as multinomial
    // takes them), handed to the engine in runs of at most one context; the generator is then
    // advanced by exactly the draws used.
    // sample_next masks only for 0 < top_k < vocab: any other top_k keeps every entry (the engine's top_k 0)
    device::gpt_engine_set_sampling(engine.handle, options.temperature,
                                    sampled && options.top_k > 0 ? options.top_k : 0);
    const std::int64_t run = config.max_positions + 1;
    const auto hand_over = [&](std::int64_t picks) {
        if (sampled) {
            const std::vector<double> draws = device_peek_uniforms(picks);
            device::gpt_engine_set_uniforms(engine.handle, draws.data(), picks);
        }
    };
    const auto used = [&](std::int64_t picks) {
        if (sampled) device_take_uniforms(picks);
    };
    const std::int64_t first_run = options.on_token ? 1 : std::min(options.max_new_tokens, run);
    hand_over(first_run);
    std::vector<std::int64_t> generated{device::gpt_engine_prefill(engine.handle, ids, length)};
    // on_token sees each token as sample_next returns it: a [1, 1] int64 tensor on the device.
    const auto emit = [&](std::int64_t token) {
        return !options.on_token || options.on_token(from_vector<std::int64_t>({token}, {1, 1}).to(prompt.device()));
    };
    if (options.on_token) {
        used(1);
        bool more = emit(generated.back());
        while (more && static_cast<std::int64_t>(generated.size()) < options.max_new_tokens) {
            std::int64_t token = 0;
            hand_over(1);
            device::gpt_engine_decode(engine.handle, 1, &token);
            used(1);
            generated.push_back(token);
            more = emit(token);
        }
    } else {
        generated.resize(static_cast<std::size_t>(options.max_new_tokens));
        std::int64_t done = 1, budget = first_run - 1;  // picks left in the current run of draws
        while (done < options.max_new_tokens) {
            if (budget == 0) {
                used(run);
                budget = std::min(options.max_new_tokens - done, run);
                hand_over(budget);
            }
            const std::int64_t n = std::min(budget, options.max_new_tokens - done);
            device::gpt_engine_decode(engine.handle, n, generated.data() + done);
            done += n;
            budget -= n;
        }
        used(options.max_new_tokens - (options.max_new_tokens - 1) / run * run);
    }
    const Tensor tail =
        from_vector<std::int64_t>(generated, {1, static_cast<std::int64_t>(generated.size())}).to(prompt.device());
    return cat({prompt, tail}, 1);
}

"""

INDEX_LINE_HELPER = """// MI355X: indices that are one line broadcast over the other dims (every stride 0 but the
// indexed dim's: index_select's and index_add_'s expanded 1-D indices) are range-checked on the
// line itself, min and max in one device call and one sync, and handed to the kernel in place
// (broadcast strides and all), instead of as a contiguous copy of the broadcast whose max and
// min are read back one at a time. The line holds every value the broadcast does (the broadcast
// is not empty), so the check passes and fails as kael's, max first. Returns the indices' first
// element, or nullptr for any other indices (kael's path).
const std::int64_t* checked_index_line(const Tensor& indices, std::size_t position, std::int64_t size,
                                       const char* op) {
    if (indices.device() == Device::CPU || indices.dtype() != DType::I64 || indices.numel() == 0) {
        return nullptr;
    }
    for (std::size_t d = 0; d < indices.shape().size(); ++d) {
        if (d != position && indices.shape()[d] != 1 && indices.strides()[d] != 0) {
            return nullptr;
        }
    }
    const auto* line = reinterpret_cast<const std::int64_t*>(indices.device_data());
    std::int64_t bounds[2];
    device::index_bounds(line, indices.shape()[position], indices.strides()[position], bounds);
    detail::checked_index(bounds[1], size, op);
    detail::checked_index(bounds[0], size, op);
    return line;
}

"""

GATHER_LINE_BRANCH = """        if (const std::int64_t* line = checked_index_line(indices, position, t.shape()[position], "gather")) {
            device::gather(t.dtype(), gathered.device_data(), t.device_data(), line,
                           detail::index_layout(t, indices, gathered, position));
            autograd::record_gather(gathered, t, dim, indices);
            return gathered;
        }
"""

SCATTER_LINE_BRANCH = """        if (const std::int64_t* line = checked_index_line(indices, position, shape()[position], "scatter_add_")) {
            device::scatter_add(dtype(), device_data(), line, source.device_data(),
                                detail::index_layout(*this, indices, source, position));
            impl_->storage->bump_version();
            return *this;
        }
"""

TARGET_BOUNDS = """    // MI355X: the targets' max and min of a device tensor in one call and one sync.
    std::int64_t bounds[2];
    if (targets.device() != Device::CPU && (targets.is_contiguous() || targets.dim() == 1)) {
        device::index_bounds(reinterpret_cast<const std::int64_t*>(targets.device_data()), targets.numel(),
                             targets.is_contiguous() ? 1 : targets.strides()[0], bounds);
    } else {
        bounds[1] = %(ns)smax(targets).item<std::int64_t>();
        bounds[0] = %(ns)smin(targets).item<std::int64_t>();
    }
    const auto largest = bounds[1];
    const auto smallest = bounds[0];
"""

ATTENTION_HELPER = """
// MI355X: the attention of CausalSelfAttention::forward without a KV cache or dropout, for f32
// heads of 64, as one device call over the fused projection's output parts [B, T, 3, H, D]
// (contiguous): the output comes back with the heads merged ([B, T, H * D], what
// transpose(1, 2).contiguous() gives), and one node takes the whole chain's backward (one
// launch writing the q, k and v gradients into one [B, T, 3, H, D] tensor) instead of the
// products, scale, mask, softmax, merge copy and three select gradients. nullopt for any other
// case, which keeps kael's ops.
std::optional<Tensor> device_causal_attention(const Tensor& parts, std::int64_t heads, std::int64_t head_dim) {
    if (parts.device() == Device::CPU || parts.dtype() != DType::F32 || head_dim != 64 || parts.numel() == 0 ||
        !parts.is_contiguous() || reinterpret_cast<std::uintptr_t>(parts.device_data()) % 16 != 0) {
        return std::nullopt;
    }
    const std::int64_t batch = parts.size(0);
    const std::int64_t length = parts.size(1);
    Tensor out = empty({batch, length, heads * head_dim}, DType::F32, parts.device());
    const Tensor lse = empty({batch, heads, length}, DType::F32, parts.device());
    device::causal_attention(DType::F32, out.device_data(), lse.device_data(), parts.device_data(), batch, length,
                             heads, head_dim);
    if (autograd::should_record(out, {&parts})) {
        autograd::set_history(
            out, "CausalAttentionBackward", {parts},
            {[saved_qkv = autograd::SavedTensor(parts), saved_out = autograd::SavedTensor(out), lse,
              shape = parts.shape(), batch, length, heads, head_dim](const Tensor& g) {
                Tensor gc = g.contiguous();
                if (reinterpret_cast<std::uintptr_t>(gc.device_data()) % 16 != 0) {
                    gc = g.clone();
                }
                Tensor dqkv = empty(shape, DType::F32, g.device());
                device::causal_attention_backward(DType::F32, dqkv.device_data(), gc.device_data(),
                                                  saved_qkv.get().device_data(), saved_out.get().device_data(),
                                                  lse.device_data(), batch, length, heads, head_dim);
                return dqkv;
            }});
    }
    return out;
}
"""

CACHED_ATTENTION_HELPER = """
// MI355X: the attention of CausalSelfAttention::forward with a KV cache when no gradient is
// recorded (generation), for f32 heads of 64: one device call reads the new queries (a view of the
// fused projection) and the keys and values (the cache's concatenated tensors, or at the first
// step the views themselves) in place and returns the heads merged ([B, T, H * D]), instead of
// the two products, scale, mask, softmax and merge copy. nullopt for any other case, which keeps
// kael's ops.
std::optional<Tensor> device_cached_attention(const Tensor& queries, const Tensor& keys, const Tensor& values,
                                              std::int64_t head_dim) {
    for (const Tensor* t : {&queries, &keys, &values}) {
        if (t->device() == Device::CPU || t->dtype() != DType::F32 || t->dim() != 4 || t->size(3) != head_dim ||
            t->strides()[3] != 1 || t->numel() == 0 || (autograd::GradMode::is_enabled() && t->requires_grad())) {
            return std::nullopt;
        }
    }
    const std::int64_t batch = queries.size(0);
    const std::int64_t heads = queries.size(1);
    const std::int64_t length = queries.size(2);
    const std::int64_t total = keys.size(2);
    if (head_dim != 64 || values.size(2) != total || total < length || keys.size(0) != batch ||
        values.size(0) != batch || keys.size(1) != heads || values.size(1) != heads) {
        return std::nullopt;
    }
    const std::int64_t qs[3] = {queries.strides()[0], queries.strides()[1], queries.strides()[2]};
    const std::int64_t ks[3] = {keys.strides()[0], keys.strides()[1], keys.strides()[2]};
    const std::int64_t vs[3] = {values.strides()[0], values.strides()[1], values.strides()[2]};
    Tensor out = empty({batch, length, heads * head_dim}, DType::F32, queries.device());
    device::cached_attention(DType::F32, out.device_data(), queries.device_data(), qs, keys.device_data(), ks,
                             values.device_data(), vs, batch, heads, length, total, head_dim);
    return out;
}
"""

CACHED_ATTENTION_BRANCH = """    if (cache != nullptr && (dropout_ == 0.0 || !is_training())) {
        if (std::optional<Tensor> mixed = device_cached_attention(queries, keys, values, head_dimension_)) {
            const Tensor output = projection_->forward(mixed->view({batch, length, dimension_}));
            return functional::dropout(output, dropout_, is_training());
        }
    }
"""

ATTENTION_BRANCH = """    if (cache == nullptr && (dropout_ == 0.0 || !is_training())) {
        if (std::optional<Tensor> mixed = device_causal_attention(parts, heads_, head_dimension_)) {
            const Tensor output = projection_->forward(mixed->view({batch, length, dimension_}));
            return functional::dropout(output, dropout_, is_training());
        }
    }
"""

GENERATE_BRANCH = """    if (auto out = device_generate(model, prompt, options)) {
        return *out;
    }
"""

# (relative path, anchor line(s), where, text). where: "before", "after", "replace", "append".
DROPOUT_HELPER = """// MI355X: dropout of a contiguous f32 / f64 device tensor with its bernoulli mask drawn on the
// device from this generator: one launch writes the output and the mask, and the generator comes
// back advanced by exactly numel() draws, as bernoulli's host draws advance it. The backward pass
// is kael's for input * mask / keep: (g / keep) * mask. nullopt for any other tensor, which keeps
// kael's ops.
std::optional<Tensor> device_dropout(const Tensor& input, double keep) {
    if (input.device() == Device::CPU || !input.is_contiguous() ||
        (input.dtype() != DType::F32 && input.dtype() != DType::F64)) {
        return std::nullopt;
    }
    Tensor out = empty(input.shape(), input.dtype(), input.device());
    Tensor mask = empty(input.shape(), input.dtype(), input.device());
    if (input.numel() > 0) {
        std::array<std::uint64_t, 313> state{};  // libstdc++'s stream form: 312 words, then the position
        const auto lock = lock_generator();
        std::stringstream words;
        words << global_generator();
        for (std::uint64_t& word : state) {
            words >> word;
        }
        device::dropout(input.dtype(), out.device_data(), mask.device_data(), input.device_data(), input.numel(),
                        keep, state.data());
        std::stringstream advanced;
        for (const std::uint64_t word : state) {
            advanced << word << ' ';
        }
        advanced >> global_generator();
    }
    if (autograd::should_record(out, {&input})) {
        autograd::set_history(out, "DropoutBackward", {input},
                              {[mask, keep](const Tensor& g) { return (g / keep) * mask; }});
    }
    return out;
}

"""

UNIFORMS_HELPER = """// MI355X: the uniform draws multinomial would take from this generator (one
// uniform_real_distribution<double>(0, 1) value per sample), for the decode engine's device
// sampler: device_peek_uniforms returns the next `count` without advancing the generator, and
// device_take_uniforms(used) then advances it by the draws the sampled picks used.
std::vector<double> device_peek_uniforms(std::int64_t count) {
    const auto lock = lock_generator();
    std::mt19937_64 copy = global_generator();
    std::uniform_real_distribution<double> uniform(0.0, 1.0);
    std::vector<double> values(static_cast<std::size_t>(count));
    for (double& value : values) {
        value = uniform(copy);
    }
    return values;
}

void device_take_uniforms(std::int64_t used) {
    const auto lock = lock_generator();
    std::uniform_real_distribution<double> uniform(0.0, 1.0);
    for (std::int64_t i = 0; i < used; ++i) {
        (void)uniform(global_generator());
    }
}

"""

UNIFORMS_DECLARATION = """
namespace kael {
// MI355X: defined beside the generator in src/random.cpp.
std::vector<double> device_peek_uniforms(std::int64_t count);
void device_take_uniforms(std::int64_t used);
} // namespace kael
"""

DROPOUT_DECLARATION = """
#include <optional>

namespace kael {
// MI355X: defined beside the generator in src/random.cpp.
std::optional<Tensor> device_dropout(const Tensor& input, double keep);
} // namespace kael
"""

DROPOUT_BRANCH = """    if (std::optional<Tensor> out = device_dropout(input, keep)) {
        return *out;
    }
"""

EDITS = [
    ("include/kael/device_kernels.h", None, "append", '\n#include "kd_kael_extensions.h"\n'),
    ("src/ops/nn.cpp", '#include "kael/ops.h"\n', "after", '#include "kael/device_kernels.h"\n'),
    ("src/ops/nn.cpp", "        const Tensor exponentials = exp(shifted_by_max(x, dim));\n", "before",
     SOFTMAX_BRANCH % "false"),
    ("src/ops/nn.cpp", "        const Tensor shifted = shifted_by_max(x, dim);\n", "before", SOFTMAX_BRANCH % "true"),
    ("src/ops/nn.cpp", "        if (x.device() != Device::CPU) {\n            Dims dims;\n", "before", STANDARDIZE_BRANCH),
    ("src/ops/nn.cpp",
     "    if (logits.device() != Device::CPU) {\n"
     "        return -gather(log_softmax(logits, 1), 1, targets.unsqueeze(1)).squeeze(1);\n    }\n",
     "replace", CROSS_ENTROPY_BRANCH),
    ("src/ops/nn.cpp", "    const Tensor weights = scale.contiguous();\n", "after", CROSS_ENTROPY_GRAD_BRANCH),
    ("src/autograd/functions_math.cpp",
     "                      [saved = SavedTensor(x), approximate](const Tensor& g) {\n", "after", GELU_BACKWARD_BRANCH),
    ("src/ops/linalg.cpp", "Tensor multiply_batches(const Tensor& a, const Tensor& b, const Shape& batch,\n", "before",
     STRIDES_HELPER),
    ("src/ops/linalg.cpp", "    const Tensor flat_a = as_batch_of_matrices(a.to(dtype), batch, rows, inner);\n", "before",
     MATMUL_BRANCH),
    ("src/optim/optimizer.cpp", '#include "kael/ops.h"\n', "after",
     '#include "kael/device_kernels.h"\n#include "kael/tensor_impl.h"\n'),
    ("src/optim/optimizer.cpp",
     "        Tensor gradient =\n            options_.weight_decay > 0.0 ? *stored + parameter * options_.weight_decay : *stored;\n",
     "before", SGD_BRANCH),
    ("src/optim/optimizer.cpp", "#include <utility>\n", "after", "#include <unordered_set>\n#include <vector>\n"),
    ("src/optim/optimizer.cpp", "void AdamBase::update() {\n", "after", ADAM_PENDING),
    ("src/optim/optimizer.cpp",
     "        const double second_correction = 1.0 - std::pow(options_.beta2, step);\n", "after", ADAM_BRANCH),
    ("src/optim/optimizer.cpp", "                       learning_rate());\n    }\n", "after", "    flush();\n"),
    ("src/autograd/functions_linalg.cpp",
     "                     const Tensor gradient = matmul(left.get().mT(), layout.matrix_gradient(g));\n", "before",
     WEIGHT_GRADIENT_BRANCH),
    ("src/autograd/functions_linalg.cpp",
     "                     const Tensor gradient = matmul(layout.matrix_gradient(g), right.get().mT());\n", "before",
     LEFT_WEIGHT_GRADIENT_BRANCH),
    ("src/ops/indexing.cpp", "Tensor masked_fill(const Tensor& t, const Tensor& mask, Scalar value) {\n", "after",
     MASKED_FILL_BRANCH),
    ("src/nn/layers.cpp", '#include "kael/ops.h"\n', "after",
     '#include "kael/autograd/grad_mode.h"\n#include "kael/device_kernels.h"\n\n#include <memory>\n#include <optional>\n\n'
     '#include "record.h"\n#include "recording.h"\n'),
    ("src/nn/layers.cpp", "    const Tensor product = matmul(input, weight_.T());\n", "before", LINEAR_BRANCH),
    ("src/nn/layers.cpp",
     "    return kael::standardize(input, static_cast<std::int64_t>(count), eps_) * weight_ + bias_;\n", "before",
     LAYER_NORM_BRANCH),
    ("src/autograd/node.cpp", '#include "kael/ops.h"\n', "after", '#include "kael/tensor_impl.h"\n'),
    ("src/autograd/node.cpp", "GradientList AccumulateGrad::apply(const Tensor& gradient) {\n", "after",
     ACCUMULATE_BRANCH),
    ("src/ops/reduce.cpp", "#include <functional>\n", "after", "#include <optional>\n"),
    ("src/ops/reduce.cpp", "Tensor device_reduce(const Reduction& reduction, device::ReduceOp op, DType dtype) {\n",
     "before", LEADING_REDUCE_HELPER),
    ("src/ops/reduce.cpp", "Tensor device_sum(const Tensor& t, const Dims& dims, bool keepdim) {\n", "after",
     LEADING_SUM_BRANCH),
    ("src/ops/reduce.cpp", "Tensor device_norm(const Tensor& t, const Dims& dims, bool keepdim) {\n", "before",
     REDUCE_HELPERS),
    ("src/ops/reduce.cpp", "Tensor prod(const Tensor& t, const Dims& dims, bool keepdim) {\n", "after", PROD_BRANCH),
    ("src/ops/reduce.cpp", "Tensor all(const Tensor& t, const Dims& dims, bool keepdim) {\n", "after",
     LOGICAL_BRANCH % "All"),
    ("src/ops/reduce.cpp", "Tensor any(const Tensor& t, const Dims& dims, bool keepdim) {\n", "after",
     LOGICAL_BRANCH % "Any"),
    ("src/ops/reduce.cpp", "Tensor argmax(const Tensor& t) {\n", "after",
     ARG_BRANCH % ("t.flatten(), {0}, false", "true", '"argmax"')),
    ("src/ops/reduce.cpp", "Tensor argmax(const Tensor& t, std::int64_t dim, bool keepdim) {\n", "after",
     ARG_BRANCH % ("t, {dim}, keepdim", "true", '"argmax"')),
    ("src/ops/reduce.cpp", "Tensor argmin(const Tensor& t) {\n", "after",
     ARG_BRANCH % ("t.flatten(), {0}, false", "false", '"argmin"')),
    ("src/ops/reduce.cpp", "Tensor argmin(const Tensor& t, std::int64_t dim, bool keepdim) {\n", "after",
     ARG_BRANCH % ("t, {dim}, keepdim", "false", '"argmin"')),
    ("src/autograd/functions_reduce.cpp", "#include <algorithm>\n", "after", "#include <optional>\n"),
    ("src/autograd/functions_reduce.cpp", '#include "kael/ops.h"\n', "after", '#include "kael/device_kernels.h"\n'),
    ("src/autograd/functions_reduce.cpp", "Dims resolved_dims(const Shape& shape, const Dims& dims) {\n", "before",
     ROW_BACKWARD_HELPERS),
    ("src/autograd/functions_reduce.cpp",
     "                        return y.get() * (g - kael::sum(g * y.get(), {dim}, true));\n", "before",
     SOFTMAX_BACKWARD_BRANCH % "false"),
    ("src/autograd/functions_reduce.cpp",
     "                        return g - kael::exp(y.get()) * kael::sum(g, {dim}, true);\n", "before",
     SOFTMAX_BACKWARD_BRANCH % "true"),
    ("src/autograd/functions_reduce.cpp",
     "                const Tensor scale = kael::sqrt(kael::var(saved.get(), dims, true, 0) + eps);\n", "before",
     STANDARDIZE_BACKWARD_BRANCH),
    ("src/nn/transformer.cpp", "#include <map>\n", "after", "#include <optional>\n#include <vector>\n"),
    ("src/nn/transformer.cpp", '#include "kael/autograd/grad_mode.h"\n', "after", '#include "kael/device_kernels.h"\n'),
    ("src/nn/transformer.cpp", "class TrainingModeRestorer {\n", "before", GENERATE_HELPER),
    ("src/nn/transformer.cpp", '#include "kael/random.h"\n', "after", '\n#include "recording.h"\n' + UNIFORMS_DECLARATION),
    ("src/nn/transformer.cpp", "constexpr double kInitialStd = 0.02;\n", "after", ATTENTION_HELPER + CACHED_ATTENTION_HELPER),
    ("src/nn/transformer.cpp",
     "        query_key_value_->forward(input).view({batch, length, 3, heads_, head_dimension_});\n", "after",
     ATTENTION_BRANCH),
    ("src/nn/transformer.cpp", "    const std::int64_t context = model.config().max_positions;\n", "after",
     GENERATE_BRANCH),
    ("src/nn/transformer.cpp", "    if (future_mask_.device() != input.device()) {\n", "before",
     CACHED_ATTENTION_BRANCH),
    ("src/ops/sequence.cpp", '#include "kael/ops.h"\n', "after", '#include "kael/device_kernels.h"\n'),
    ("src/ops/sequence.cpp", "        return t.to(dtype).clone();\n    }\n", "after", CUMSUM_BRANCH),
    ("src/ops/indexing.cpp", '#include "kael/kernels.h"\n', "after", '#include "kael/device_kernels.h"\n'),
    ("src/ops/indexing.cpp", "namespace kael {\n\nnamespace {\n", "after", INDEX_LINE_HELPER),
    ("src/ops/indexing.cpp",
     "        const Tensor flat = autograd::without_grad([&] { return indices.contiguous(); });\n"
     "        detail::check_device_indices(flat, t.shape()[position], \"gather\");\n", "before", GATHER_LINE_BRANCH),
    ("src/ops/inplace.cpp", '#include "kael/kernels.h"\n', "after", '#include "kael/device_kernels.h"\n'),
    ("src/ops/inplace.cpp", "namespace kael {\n\nnamespace {\n", "after", INDEX_LINE_HELPER),
    ("src/ops/inplace.cpp", "        const Tensor contiguous_indices = indices.contiguous();\n"
     "        detail::check_device_indices(contiguous_indices, shape()[position], \"scatter_add_\");\n", "before",
     SCATTER_LINE_BRANCH),
    ("src/ops/nn.cpp", "    const auto largest = max(targets).item<std::int64_t>();\n"
     "    const auto smallest = min(targets).item<std::int64_t>();\n", "replace", TARGET_BOUNDS % {"ns": ""}),
    ("src/nn/loss.cpp", '#include "kael/ops.h"\n', "after", '#include "kael/device_kernels.h"\n'),
    ("src/nn/loss.cpp", "    const auto largest = kael::max(targets).item<std::int64_t>();\n"
     "    const auto smallest = kael::min(targets).item<std::int64_t>();\n", "replace", TARGET_BOUNDS % {"ns": "kael::"}),
    ("src/random.cpp", '#include "kael/ops.h"\n', "after",
     '#include "kael/device_kernels.h"\n\n#include <array>\n#include <optional>\n#include <sstream>\n\n'
     '#include "recording.h"\n'),
    ("src/random.cpp", "Tensor multinomial(const Tensor& weights, std::int64_t samples, bool replacement) {\n", "before",
     DROPOUT_HELPER + UNIFORMS_HELPER),
    ("src/nn/functional.cpp", '#include "kael/random.h"\n', "after", DROPOUT_DECLARATION),
    ("src/nn/functional.cpp", "    const double keep = 1.0 - p;\n", "after", DROPOUT_BRANCH),
]


def apply(ref: Path, out: Path) -> list[Path]:
    texts: dict[str, str] = {}
    for rel, anchor, where, text in EDITS:
        body = texts.get(rel)
        if body is None:
            body = (ref / rel).read_text()
        if where == "append":
            body = body + text
        else:
            count = body.count(anchor)
            if count != 1:
                raise SystemExit(f"{rel}: anchor found {count} times (expected 1): {anchor!r}")
            if where == "before":
                body = body.replace(anchor, text + anchor)
            elif where == "after":
                body = body.replace(anchor, anchor + text)
            else:
                body = body.replace(anchor, text)
        texts[rel] = body
    written = []
    for rel, body in texts.items():
        target = out / rel
        target.parent.mkdir(parents=True, exist_ok=True)
        if not target.is_file() or target.read_text() != body:
            target.write_text(body)
        written.append(target)
    return written


if __name__ == "__main__":
    if len(sys.argv) != 3:
        raise SystemExit(__doc__)
    for path in apply(Path(sys.argv[1]), Path(sys.argv[2])):
        print(path)
