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

    std::printf("%d of %d cases passed\n", cases - failures + (panicked ? 1 : 0), cases + 1);
    return failures == 0 ? 0 : 1;
}
