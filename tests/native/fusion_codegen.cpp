// Host-only check of the fusion code generator: builds lazy graphs over
// storage-less device leaves (no GPU needed), asks the backend for the kernel
// source each graph would compile to, and compiles it with hipRTC for gfx950.
// Covers elementwise regions (float4 and indexed paths, float32 and float64)
// and row regions (softmax, reductions of broadcast chains, 3-d rows).
#include <hip/hiprtc.h>

#include <cstdio>
#include <memory>
#include <string>

#include "lmp_hip.h"
#include "ops.hpp"

namespace lmp::tensor::hip {
std::string fused_source_for(TensorImpl* root);
std::string fused_group_source_for(const std::vector<TensorImpl*>& roots);
}

using namespace lmp::tensor;
using P = std::shared_ptr<TensorImpl>;

namespace {

int failures = 0;

// Graphs are built in statements of their own before check() runs: a
// temporary still alive during check() would own an interior node, which the
// backend then realises separately (and that needs a device).
P leaf(std::vector<size_t> shape, DataType dt = DataType::Float32) {
  return std::make_shared<TensorImpl>(Storage(0, DeviceType::HIP), shape, dt);
}
P bin(int op, const P& a, const P& b) { return lazy::record(lazy::make_binary(op, a, b)); }
P un(int op, const P& a) { return lazy::record(lazy::make_unary(op, a)); }
P red(int op, const P& a) {
  return lazy::record(lazy::make_reduce(op, a, a->shape().size() - 1));
}

void check_source(const char* what, const std::string& src, const char* must_contain) {
  if (src.find(must_contain) == std::string::npos) {
    std::printf("FAIL %s: source lacks \"%s\"\n", what, must_contain);
    ++failures;
    return;
  }
  hiprtcProgram prog;
  hiprtcCreateProgram(&prog, src.c_str(), "lmp_fused.hip", 0, nullptr, nullptr);
  const char* opts[] = {"--offload-arch=gfx950", "-O3", "-ffp-contract=off", "-std=c++17"};
  const hiprtcResult r = hiprtcCompileProgram(prog, 4, opts);
  if (r != HIPRTC_SUCCESS) {
    size_t n = 0;
    hiprtcGetProgramLogSize(prog, &n);
    std::string log(n, '\0');
    if (n) hiprtcGetProgramLog(prog, log.data());
    std::printf("FAIL %s: hipRTC: %s\n%s\n", what, hiprtcGetErrorString(r), log.c_str());
    ++failures;
  } else {
    std::printf("ok   %s (%zu bytes)\n", what, src.size());
  }
  hiprtcDestroyProgram(&prog);
}

void check(const char* what, const P& root, const char* must_contain) {
  check_source(what, hip::fused_source_for(root.get()), must_contain);
}

P fill(std::vector<size_t> shape, double v) {
  return lazy::record(lazy::make_fill(shape, DeviceType::HIP, DataType::Float32, v));
}

P softmax(P x) {
  P m = red(LMP_RED_MAX, x);
  P e = un(LMP_UN_EXP, bin(LMP_BIN_SUB, x, m));
  return bin(LMP_BIN_DIV, e, red(LMP_RED_SUM, e));
}

}  // namespace

int main() {
  std::setvbuf(stdout, nullptr, _IONBF, 0);
  {
    P a = leaf({8192, 64}), b = leaf({8192, 1});
    const P r = bin(LMP_BIN_ADD, bin(LMP_BIN_MUL, a, a), b);
    check("a*a+b float4", r, "lmp_v4");
  }
  {
    P a = leaf({4, 1, 3}), b = leaf({1, 5, 3});
    const P r = bin(LMP_BIN_MUL, a, b);
    check("3-d broadcast indexed", r, "rest");
  }
  {
    P a = leaf({257, 64}, DataType::Float64), b = leaf({257, 1}, DataType::Float64);
    const P r =
        bin(LMP_BIN_SUB, bin(LMP_BIN_MUL, un(LMP_UN_EXP, a), b),
            bin(LMP_BIN_DIV, lazy::record(lazy::make_unary(LMP_UN_CLAMP, a, 0.0, 1e300)), b));
    check("float64 chain", r, "exp(");
  }
  {
    const P r1 = softmax(leaf({512, 1000}));
    check("softmax 512x1000 (float4 order)", r1, "lmp_swap<32>");
    const P r2 = softmax(leaf({32, 10}));
    check("softmax 32x10 (scalar order)", r2, "lmp_swap<32>");
    const P r3 = softmax(leaf({7, 333}));
    check("softmax 7x333", r3, "lmp_swap<32>");
    const P r4 = softmax(leaf({64, 100}, DataType::Float64));
    check("softmax float64", r4, "double");
  }
  for (int op : {LMP_RED_SUM, LMP_RED_MAX, LMP_RED_MIN, LMP_RED_PROD}) {
    P a = leaf({5, 3, 12}), w = leaf({12}), c = leaf({1});
    const P r = red(op, bin(LMP_BIN_ADD, bin(LMP_BIN_MUL, a, w), c));
    check("reduce of a*w+c, 3-d rows", r, "lmp_swap<32>");
  }
  {
    P p = leaf({32, 10}), y = leaf({32, 10}), k = leaf({1});
    const P r = red(LMP_RED_SUM, bin(LMP_BIN_MUL, un(LMP_UN_NEG, y),
                                     un(LMP_UN_LOG, bin(LMP_BIN_ADD, p, k))));
    check("loss row", r, "logf(");
  }
  {
    // Interior values something else holds become extra outputs of the
    // region's kernel (xo0, ..) instead of separate realisations.
    P a = leaf({64, 128}), b = leaf({64, 128});
    const P t = bin(LMP_BIN_MUL, a, b);  // held below: stored by the kernel
    const P r = bin(LMP_BIN_SUB, bin(LMP_BIN_ADD, t, a), b);
    check("held interior value as extra output (float4)", r, "xo0");
    P c = leaf({64, 100});
    const P e = un(LMP_UN_EXP, c);  // held
    const P s = red(LMP_RED_SUM, e);
    check("held interior value in a row kernel", s, "xo0");
  }
  {
    // A row region taking a [1, 1] constant (the loss seed) and the backward
    // functors of abs and clamp.
    P x = leaf({32, 10}), g = leaf({32, 10});
    const P seed = fill({1, 1}, 1.0);
    const P r = red(LMP_RED_SUM,
                    bin(LMP_BIN_MUL, seed,
                        lazy::record(lazy::make_binary(LMP_BIN_CLAMP_BACKWARD, x, g, 0.0, 1e300))));
    check("row region with a [1,1] fill and clamp backward", r, "__uint_as_float(0x3f800000u)");
    const P ab = lazy::record(lazy::make_binary(LMP_BIN_ABS_BACKWARD, x, g));
    check("abs backward", ab, "(-");
  }
  {
    // realize_all's grouped kernel: float4, indexed and float64 regions, each
    // in its own workgroup range.
    P p1 = leaf({256, 64}), g1 = leaf({256, 64}), lr = leaf({1});
    P p2 = leaf({10}), g2 = leaf({10});
    P p3 = leaf({33, 7}, DataType::Float64), g3 = leaf({33, 7}, DataType::Float64),
      lr64 = leaf({1}, DataType::Float64);
    const P u1 = bin(LMP_BIN_SUB, p1, bin(LMP_BIN_MUL, lr, g1));
    const P u2 = bin(LMP_BIN_SUB, p2, bin(LMP_BIN_MUL, lr, g2));
    const P u3 = bin(LMP_BIN_SUB, p3, bin(LMP_BIN_MUL, lr64, g3));
    check_source("grouped updates (float4, indexed, float64)",
                 hip::fused_group_source_for({u1.get(), u2.get(), u3.get()}),
                 "else if (blockIdx.x <");
  }
  if (failures) {
    std::printf("%d codegen failures\n", failures);
    return 1;
  }
  std::printf("fusion codegen ok\n");
  return 0;
}
