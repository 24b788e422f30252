// suite_main.cpp -- driver for the reference's autograd, convolution and
// Transformer unit tests (its tests/test_autograd.cpp, test_conv.cpp and
// test_transformer.cpp, compiled in place against this repository's engine
// headers). The reference's own driver also runs suites that need tensor
// slicing and axis maxima, Sigmoid / Tanh / GELU and its CUDA control header,
// which this engine does not provide, so this one runs the three suites that
// need none of them and reports their counters from test_support.hpp.
#include <cstdio>

#include "test_support.hpp"

int main() {
    run_autograd_tests();
    run_conv_tests();
    run_transformer_tests();
    std::printf("\nreference suites: %d checks, %d failed\n", testing::g_checks,
                testing::g_failures);
    return testing::g_failures == 0 ? 0 : 1;
}
