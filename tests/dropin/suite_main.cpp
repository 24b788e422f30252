// suite_main.cpp -- driver for the reference's unit suites (its tests/test_tensor.cpp,
// test_autograd.cpp, test_nn.cpp, test_conv.cpp, test_transformer.cpp and
// test_reference.cpp), compiled in place against this repository's engine headers. The
// reference's own driver also runs the CUDA indexing suite, which needs its CUDA control
// header; this one runs the other six in the same order and reports their counters from
// test_support.hpp.
#include <cstdio>

#include "test_support.hpp"

int main() {
    run_tensor_tests();
    run_autograd_tests();
    run_nn_tests();
    run_conv_tests();
    run_transformer_tests();
    run_reference_tests();
    std::printf("\nreference suites: %d checks, %d failed\n", testing::g_checks,
                testing::g_failures);
    return testing::g_failures == 0 ? 0 : 1;
}
