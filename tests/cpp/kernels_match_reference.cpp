// The reference's GPU parity test, restated over the C++ host mirror:
// crates/staleynet-cuda/tests/kernels_match_reference.rs:54-91,
// `matmul_matches_reference_for_every_storage_and_kernel`. Every kernel
// against the CPU reference (the oracle in oracle/matmul_oracle.c), ragged
// sizes x batch {1, 3} x {NN, TN, NT, TT}, scale 0.7, accumulate onto random
// values, relative error below the kernel's tolerance. Also the reference's
// shared-GPU pattern and the panic on an undersized operand
// (ops/matmul.rs:147-149). Exit status 0 when every case passes.
#include <cmath>
#include <cstdio>
#include <cstdint>
#include <tuple>
#include <vector>

#include "staleynet_cuda.hpp"

// The oracle's C entry points (oracle/matmul_oracle.c; test infrastructure).
extern "C" {
void oracle_matmul(size_t rows, size_t cols, size_t inner, int left_t, int right_t, size_t count, size_t batch_left,
                   size_t batch_right, size_t batch_output, float scale, int accumulate, const float* left,
                   const float* right, float* output);
void oracle_random_values(size_t count, uint64_t seed, float* out);
float oracle_relative_error(const float* expected, const float* actual, size_t n);
void oracle_add_row_bias(float* output, size_t rows, size_t cols, const float* bias);
void oracle_accumulate_column_sums(const float* input, size_t rows, size_t cols, float* sums, float* scratch);
void oracle_causal_softmax(float* scores, size_t total_rows, size_t queries, size_t keys, float scale,
                           size_t query_offset);
void oracle_softmax_backward(const float* probabilities, float* grad, size_t rows, size_t cols);
void oracle_cross_entropy(const float* logits, const uint32_t* targets, size_t rows, size_t cols, size_t column_offset,
                          size_t classes, size_t target_stride, size_t target_offset, float grad_scale, float* losses,
                          float* grad);
void oracle_split_heads(const float* packed, float* head_major, const size_t* layout);
void oracle_merge_heads(const float* head_major, float* packed, const size_t* layout);
}

using namespace staleynet_cuda;

namespace {

std::vector<float> random_values(size_t count, uint64_t seed) {
    std::vector<float> out(count);
    oracle_random_values(count, seed, out.data());
    return out;
}

void reference_matmul(const MatmulSpec& spec, const std::vector<float>& left, const std::vector<float>& right,
                      std::vector<float>& output) {
    oracle_matmul(spec.rows, spec.cols, spec.inner, spec.left == Storage::Transposed,
                  spec.right == Storage::Transposed, spec.batch.count, spec.batch.left, spec.batch.right,
                  spec.batch.output, spec.scale, spec.write == WriteMode::Accumulate, left.data(), right.data(),
                  output.data());
}

float relative_error(const std::vector<float>& expected, const std::vector<float>& actual) {
    return oracle_relative_error(expected.data(), actual.data(), expected.size());
}

}  // namespace

int main() {
    Gpu gpu = Gpu::new_(0);
    gpu.bind_to_current_thread();
    const std::vector<std::tuple<size_t, size_t, size_t>> sizes = {
        {1, 1, 1}, {17, 33, 9}, {64, 48, 70}, {5, 129, 31}, {130, 197, 100}};
    const MatmulKernel kernels[] = {MatmulKernel::Naive, MatmulKernel::Tiled, MatmulKernel::Blocked,
                                    MatmulKernel::TensorCore};
    int failures = 0, cases = 0;

    for (auto [rows, cols, inner] : sizes) {
        for (size_t batch : {size_t(1), size_t(3)}) {
            const BatchStrides strides{batch, rows * inner, inner * cols, rows * cols};
            const MatmulSpec base = MatmulSpec::new_(rows, cols, inner).batched(strides).scaled(0.7f).accumulate();
            const MatmulSpec variants[] = {base, base.left_transposed(), base.right_transposed(),
                                           base.left_transposed().right_transposed()};
            for (const MatmulSpec& spec : variants) {
                const std::vector<float> left = random_values(batch * rows * inner, 1);
                const std::vector<float> right = random_values(batch * inner * cols, 2);
                const std::vector<float> initial = random_values(batch * rows * cols, 3);
                std::vector<float> expected = initial;
                reference_matmul(spec, left, right, expected);

                for (MatmulKernel kernel : kernels) {
                    gpu.matmul_kernel = kernel;
                    const Tensor left_tensor = gpu.upload(Shape::vector(left.size()), left);
                    const Tensor right_tensor = gpu.upload(Shape::vector(right.size()), right);
                    Tensor output = gpu.upload(Shape::vector(initial.size()), initial);
                    gpu.matmul(spec, left_tensor, right_tensor, output);
                    const std::vector<float> actual = gpu.download(output);
                    const float error = relative_error(expected, actual);
                    bool finite = true;
                    for (float v : actual) finite = finite && std::isfinite(v);
                    ++cases;
                    if (!(error < tolerance(kernel)) || !finite) {
                        ++failures;
                        std::printf("FAIL %s %zux%zux%zu batch %zu left %d right %d: relative error %g\n",
                                    name(kernel), rows, cols, inner, batch, int(spec.left), int(spec.right), error);
                    }
                }
            }
        }
    }

    // `assert!(left.len() >= ...)` (ops/matmul.rs:147) as a thrown Panic.
    bool panicked = false;
    try {
        const Tensor small = gpu.zeros(Shape::vector(3));
        const Tensor right = gpu.zeros(Shape::vector(4));
        Tensor out = gpu.zeros(Shape::vector(4));
        gpu.matmul(MatmulSpec::new_(2, 2, 2), small, right, out);
    } catch (const Panic& panic) {
        panicked = std::string(panic.what()) == "matmul: left operand too small";
    }
    if (!panicked) {
        ++failures;
        std::printf("FAIL undersized left operand did not panic\n");
    }

    // The bias half of `elementwise_ops_match_reference` (kernels_match_reference.rs:125-170):
    // shape 9 x 50, LCG seeds 7 (input) and 9 (bias); add_row_bias is exact, the column sums
    // within the tolerance. Then Linear::forward fused (matmul_bias) against matmul +
    // add_row_bias: the same bits.
    {
        const size_t rows = 9, cols = 50;
        const std::vector<float> input = random_values(rows * cols, 7);
        const std::vector<float> bias = random_values(cols, 9);
        std::vector<float> expected = input;
        oracle_add_row_bias(expected.data(), rows, cols, bias.data());
        Tensor combined = gpu.upload(Shape::new_(rows, cols), input);
        const Tensor bias_tensor = gpu.upload(Shape::vector(cols), bias);
        gpu.add_row_bias(combined, bias_tensor);
        ++cases;
        if (gpu.download(combined) != expected) {
            ++failures;
            std::printf("FAIL add_row_bias differs from the reference's per-element add\n");
        }
        std::vector<float> sums_expected = bias, scratch(cols);
        oracle_accumulate_column_sums(input.data(), rows, cols, sums_expected.data(), scratch.data());
        Tensor sums = gpu.upload(Shape::vector(cols), bias);
        gpu.accumulate_column_sums(gpu.upload(Shape::new_(rows, cols), input), sums);
        ++cases;
        if (!(relative_error(sums_expected, gpu.download(sums)) < tolerance(MatmulKernel::Blocked))) {
            ++failures;
            std::printf("FAIL accumulate_column_sums\n");
        }
        gpu.matmul_kernel = MatmulKernel::Blocked;
        const std::vector<float> x = random_values(130 * 100, 1), w = random_values(100 * cols, 2);
        const Tensor xt = gpu.upload(Shape::new_(130, 100), x), wt = gpu.upload(Shape::new_(100, cols), w);
        Tensor fused = gpu.zeros(Shape::new_(130, cols)), separate = gpu.zeros(Shape::new_(130, cols));
        gpu.matmul_bias(MatmulSpec::new_(130, cols, 100), xt, wt, bias_tensor, fused);
        gpu.matmul(MatmulSpec::new_(130, cols, 100), xt, wt, separate);
        gpu.add_row_bias(separate, bias_tensor);
        ++cases;
        if (gpu.download(fused) != gpu.download(separate)) {
            ++failures;
            std::printf("FAIL matmul_bias differs from matmul + add_row_bias\n");
        }
        // Linear::backward's weight and bias gradients in one call: the product's bits are matmul's,
        // and on integer inputs the column sums are exact in any order.
        {
            const size_t n = 260, k = 100, m = 132;
            std::vector<float> xi(k * m), dyi(k * n);
            for (size_t i = 0; i < xi.size(); ++i) xi[i] = float(int((i * 7919) % 33) - 16);
            for (size_t i = 0; i < dyi.size(); ++i) dyi[i] = float(int((i * 104729) % 33) - 16);
            const Tensor xg = gpu.upload(Shape::new_(k, m), xi), dyg = gpu.upload(Shape::new_(k, n), dyi);
            const MatmulSpec grad = MatmulSpec::new_(m, n, k).left_transposed().accumulate();
            Tensor dw_fused = gpu.zeros(Shape::new_(m, n)), dw_separate = gpu.zeros(Shape::new_(m, n));
            Tensor db = gpu.upload(Shape::vector(n), std::vector<float>(n, 1.f));
            gpu.matmul_column_sums(grad, xg, dyg, dw_fused, db);
            gpu.matmul(grad, xg, dyg, dw_separate);
            std::vector<float> db_expected(n, 1.f), db_scratch(n);
            oracle_accumulate_column_sums(dyi.data(), k, n, db_expected.data(), db_scratch.data());
            ++cases;
            if (gpu.download(dw_fused) != gpu.download(dw_separate)) {
                ++failures;
                std::printf("FAIL matmul_column_sums product differs from matmul\n");
            }
            ++cases;
            if (gpu.download(db) != db_expected) {
                ++failures;
                std::printf("FAIL matmul_column_sums sums differ from the row-order sums\n");
            }
        }
        bool length_panic = false;
        try {
            Tensor out = gpu.zeros(Shape::new_(rows, cols));
            gpu.add_row_bias(out, gpu.zeros(Shape::vector(cols - 1)));
        } catch (const Panic& panic) {
            length_panic = std::string(panic.what()) == "add_row_bias: bias length must equal output columns";
        }
        ++cases;
        if (!length_panic) {
            ++failures;
            std::printf("FAIL short bias did not panic\n");
        }
    }

    auto expect = [&](bool ok, const char* what) {
        ++cases;
        if (!ok) {
            ++failures;
            std::printf("FAIL %s\n", what);
        }
    };

    // `causal_softmax_and_backward_match_reference` (kernels_match_reference.rs:172-195):
    // 3 matrices of 5 queries x 70 keys, query offset 40, scale 0.5, LCG seeds 10 and 11.
    {
        const size_t matrices = 3, queries = 5, keys = 70, rows = matrices * queries;
        const std::vector<float> scores = random_values(rows * keys, 10);
        const std::vector<float> upstream = random_values(rows * keys, 11);
        std::vector<float> probabilities = scores, grad = upstream;
        oracle_causal_softmax(probabilities.data(), rows, queries, keys, 0.5f, 40);
        oracle_softmax_backward(probabilities.data(), grad.data(), rows, keys);
        Tensor p = gpu.upload(Shape::new_(rows, keys), scores);
        gpu.causal_softmax(p, queries, 0.5f, 40);
        Tensor g = gpu.upload(Shape::new_(rows, keys), upstream);
        gpu.softmax_backward(p, g);
        expect(relative_error(probabilities, gpu.download(p)) < tolerance(MatmulKernel::Blocked), "causal_softmax");
        expect(relative_error(grad, gpu.download(g)) < tolerance(MatmulKernel::Blocked), "softmax_backward");
        bool shape_panic = false;
        try {
            Tensor bad = gpu.zeros(Shape::new_(10, 8));
            gpu.causal_softmax(bad, 3, 1.0f, 0);
        } catch (const Panic& panic) {
            shape_panic = std::string(panic.what()) == "causal_softmax: rows must be a multiple of queries";
        }
        expect(shape_panic, "causal_softmax shape panic");
    }

    // `split_and_merge_heads_follow_the_layout_formula` (kernels_match_reference.rs:199-231):
    // dense(2, 5, 3, 4, 3 * 12 + 2, 13).in_cache(9, 2), LCG seed 12; bit-exact.
    {
        const HeadLayout layout = HeadLayout::dense(2, 5, 3, 4, 3 * 12 + 2, 13).in_cache(9, 2);
        const std::vector<float> packed = random_values(layout.batch * layout.time * layout.width, 12);
        const sn_head_layout l = layout.to_ffi();
        const size_t fields[8] = {l.batch, l.time, l.heads, l.head_dim, l.width, l.column_offset, l.time_capacity,
                                  l.time_offset};
        std::vector<float> head_major(layout.batch * layout.heads * layout.time_capacity * layout.head_dim, 0.f);
        oracle_split_heads(packed.data(), head_major.data(), fields);
        std::vector<float> merged(packed.size(), 0.f);
        oracle_merge_heads(head_major.data(), merged.data(), fields);
        const Tensor packed_tensor = gpu.upload(Shape::new_(layout.batch * layout.time, layout.width), packed);
        Tensor head_tensor = gpu.zeros(Shape::new_(layout.batch * layout.heads * layout.time_capacity, layout.head_dim));
        gpu.split_heads(packed_tensor, head_tensor, layout);
        expect(gpu.download(head_tensor) == head_major, "split_heads");
        Tensor merged_tensor = gpu.zeros(packed_tensor.shape());
        gpu.merge_heads(head_tensor, merged_tensor, layout);
        expect(gpu.download(merged_tensor) == merged, "merge_heads");
        bool range_panic = false;
        try {
            gpu.split_heads(packed_tensor, head_tensor, layout.in_cache(9, 5));
        } catch (const Panic& panic) {
            range_panic = std::string(panic.what()) == "HeadLayout: time range exceeds capacity";
        }
        expect(range_panic, "HeadLayout range panic");
    }

    // `cross_entropy_matches_reference` (kernels_match_reference.rs:277-298): 13 x 50 logits
    // (LCG seed 15), the head at columns 10 .. 47 with 2 targets per row (slot 1), every 7th
    // target empty, gradient scale 0.25.
    {
        const size_t rows = 13, cols = 50;
        const CrossEntropyHead head{10, 37, 2, 1, 0.25f};
        const std::vector<float> logits = random_values(rows * cols, 15);
        std::vector<uint32_t> targets(rows * 2);
        for (size_t i = 0; i < targets.size(); ++i) targets[i] = i % 7 == 0 ? SN_EMPTY_TOKEN : uint32_t(i * 5 % 37);
        std::vector<float> losses(rows, 0.f), grad(rows * cols, 0.f);
        oracle_cross_entropy(logits.data(), targets.data(), rows, cols, head.column_offset, head.classes,
                             head.target_stride, head.target_offset, head.grad_scale, losses.data(), grad.data());
        const Tensor logit_tensor = gpu.upload(Shape::new_(rows, cols), logits);
        const TokenBuffer target_buffer = gpu.upload_tokens(targets);
        Tensor loss_tensor = gpu.zeros(Shape::vector(rows));
        Tensor grad_tensor = gpu.zeros(Shape::new_(rows, cols));
        gpu.cross_entropy(logit_tensor, target_buffer, head, loss_tensor, grad_tensor);
        expect(relative_error(losses, gpu.download(loss_tensor)) < tolerance(MatmulKernel::Blocked), "cross_entropy losses");
        expect(relative_error(grad, gpu.download(grad_tensor)) < tolerance(MatmulKernel::Blocked), "cross_entropy grad");
        expect(gpu.download_tokens(target_buffer) == targets, "token round trip");
    }

    // The fused attention forward against the reference's three calls (scores product,
    // causal_softmax, mix product; layers/attention.rs:206-213): 2 heads x 70 queries x 70
    // keys x 64, scale 0.125, LCG seeds 20-22.
    {
        const size_t heads = 2, t = 70, h = 64;
        const std::vector<float> q = random_values(heads * t * h, 20), k = random_values(heads * t * h, 21),
                                 v = random_values(heads * t * h, 22);
        std::vector<float> scores(heads * t * t, 0.f), out(heads * t * h, 0.f);
        reference_matmul(MatmulSpec::new_(t, t, h).right_transposed().batched(BatchStrides{heads, t * h, t * h, t * t}),
                         q, k, scores);
        oracle_causal_softmax(scores.data(), heads * t, t, t, 0.125f, 0);
        reference_matmul(MatmulSpec::new_(t, h, t).batched(BatchStrides{heads, t * t, t * h, t * h}), scores, v, out);
        const Tensor qt = gpu.upload(Shape::new_(heads * t, h), q), kt = gpu.upload(Shape::new_(heads * t, h), k),
                     vt = gpu.upload(Shape::new_(heads * t, h), v);
        Tensor ot = gpu.zeros(Shape::new_(heads * t, h)), pt = gpu.zeros(Shape::new_(heads * t, t));
        const sn_attention_shape shape{heads, t, t, h, t * h, t * h, 0, 0.125f};
        gpu.causal_attention(qt, kt, vt, ot, shape, &pt);
        expect(relative_error(out, gpu.download(ot)) < tolerance(MatmulKernel::Blocked), "causal_attention output");
        expect(relative_error(scores, gpu.download(pt)) < tolerance(MatmulKernel::Blocked),
               "causal_attention probabilities");

        // The backward's dP product and softmax_backward (attention.rs:238-248) against the fused
        // probability gradient, on the oracle's probabilities and output; dO from LCG seed 23.
        const std::vector<float> d_out = random_values(heads * t * h, 23);
        std::vector<float> dp(heads * t * t, 0.f);
        reference_matmul(MatmulSpec::new_(t, t, h).right_transposed().batched(BatchStrides{heads, t * h, t * h, t * t}),
                         d_out, v, dp);
        oracle_softmax_backward(scores.data(), dp.data(), heads * t, t);
        const Tensor dot = gpu.upload(Shape::new_(heads * t, h), d_out), oref = gpu.upload(Shape::new_(heads * t, h), out),
                     pref = gpu.upload(Shape::new_(heads * t, t), scores);
        Tensor ds = gpu.zeros(Shape::new_(heads * t, t));
        gpu.causal_attention_score_grad(dot, vt, oref, pref, ds, shape);
        expect(relative_error(dp, gpu.download(ds)) < tolerance(MatmulKernel::Blocked), "causal_attention_score_grad");

        // Training without the probabilities: the forward with statistics gives causal_attention's O
        // bit for bit, and the backward from it gives the dQ, dK and dV products of attention.rs:250-260
        // (dp now holds dS) and :244-247 on the oracle's calls.
        std::vector<float> dq(heads * t * h, 0.f), dk(heads * t * h, 0.f), dv(heads * t * h, 0.f);
        reference_matmul(MatmulSpec::new_(t, h, t).scaled(0.125f).batched(BatchStrides{heads, t * t, t * h, t * h}),
                         dp, k, dq);
        reference_matmul(
            MatmulSpec::new_(t, h, t).left_transposed().scaled(0.125f).batched(BatchStrides{heads, t * t, t * h, t * h}),
            dp, q, dk);
        reference_matmul(MatmulSpec::new_(t, h, t).left_transposed().batched(BatchStrides{heads, t * t, t * h, t * h}),
                         scores, d_out, dv);
        Tensor o_stats = gpu.zeros(Shape::new_(heads * t, h)), stats = gpu.zeros(Shape::vector(2 * heads * t));
        gpu.causal_attention_with_stats(qt, kt, vt, o_stats, stats, shape);
        expect(gpu.download(o_stats) == gpu.download(ot), "causal_attention_with_stats output");
        Tensor dqt = gpu.zeros(Shape::new_(heads * t, h)), dkt = gpu.zeros(Shape::new_(heads * t, h)),
               dvt = gpu.zeros(Shape::new_(heads * t, h));
        gpu.causal_attention_backward(qt, kt, vt, o_stats, dot, stats, dqt, dkt, dvt, shape);
        expect(relative_error(dq, gpu.download(dqt)) < tolerance(MatmulKernel::Blocked), "causal_attention_backward dQ");
        expect(relative_error(dk, gpu.download(dkt)) < tolerance(MatmulKernel::Blocked), "causal_attention_backward dK");
        expect(relative_error(dv, gpu.download(dvt)) < tolerance(MatmulKernel::Blocked), "causal_attention_backward dV");
    }

    std::printf("%d of %d cases passed\n", cases - failures + (panicked ? 1 : 0), cases + 1);
    return failures == 0 ? 0 : 1;
}
