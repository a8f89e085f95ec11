// C++ host-API tests over libbarracuda_hip, written as the reference's own
// Rust tests are (crates/barracuda/src/ops/*.rs #[cfg(test)] modules,
// crates/barracuda/tests/fault_injection.rs), against include/barracuda_hip_ops.hpp.
//
//   bch_host_tests --cpu   validation and no-device behaviour (no GPU needed)
//   bch_host_tests --gpu   everything, on device 0
// Exit status 0 when every test passes; one line per test on stdout.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "barracuda_hip_ops.hpp"

using namespace barracuda;

namespace {

int g_fail = 0, g_pass = 0;
std::shared_ptr<HipDevice> g_dev;

#define REQUIRE(cond)                                                                   \
  do {                                                                                  \
    if (!(cond)) throw std::runtime_error(std::string("requirement failed: ") + #cond + \
                                          " (" + __FILE__ + ":" + std::to_string(__LINE__) + ")"); \
  } while (0)

void run(const char* name, const std::function<void()>& fn) {
  try {
    fn();
    ++g_pass;
    std::printf("PASS %s\n", name);
  } catch (const std::exception& e) {
    ++g_fail;
    std::printf("FAIL %s: %s\n", name, e.what());
  }
  std::fflush(stdout);
}

Tensor T(const std::vector<float>& d, std::vector<size_t> s) { return Tensor::from_vec_on(d, std::move(s), g_dev).unwrap(); }

// the reference tests' CPU matmul (ops/matmul.rs:250-262): i, j, p with mul_add
std::vector<float> matmul_cpu(const std::vector<float>& a, const std::vector<float>& b, size_t m, size_t k, size_t n) {
  std::vector<float> r(m * n, 0.0f);
  for (size_t i = 0; i < m; ++i)
    for (size_t j = 0; j < n; ++j) {
      float sum = 0.0f;
      for (size_t p = 0; p < k; ++p) sum = std::fma(a[i * k + p], b[p * n + j], sum);
      r[i * n + j] = sum;
    }
  return r;
}

bool has_shape_words(const std::string& m) {
  std::string s = m;
  for (auto& c : s) c = (char)std::tolower(c);
  return s.find("shape") != std::string::npos || s.find("dimension") != std::string::npos ||
         s.find("mismatch") != std::string::npos;
}

// ---------------------------------------------------------------- CPU-only tests
void cpu_tests() {
  run("validate_matmul_requires_2d", [] {
    auto e = MatMul::validate({4}, {4, 4});
    REQUIRE(e && e->kind == ErrorKind::InvalidOperation && e->message.find("2D+") != std::string::npos);
  });
  run("validate_matmul_inner_dim_mismatch", [] {  // fault_injection.rs:29-60
    auto e = MatMul::validate({2, 3}, {4, 2});
    REQUIRE(e && e->kind == ErrorKind::ShapeMismatch && has_shape_words(e->message));
    REQUIRE(e->message == "Shape mismatch: expected [2, 3], got [4, 2]");
    REQUIRE(!MatMul::validate({2, 3}, {3, 5}));
    REQUIRE(!MatMul::validate({2, 3, 7}, {3, 5}));  // >= 3-D uses shape[0..2] (matmul.rs:103-107)
  });
  run("validate_batch_matmul", [] {
    REQUIRE(BatchMatMul::validate({2, 2, 3}, {2, 3, 2}) == std::nullopt);
    REQUIRE(BatchMatMul::validate({2, 2, 3}, {3, 3, 2})->kind == ErrorKind::ShapeMismatch);
    REQUIRE(BatchMatMul::validate({2, 3}, {2, 3, 2})->kind == ErrorKind::InvalidOperation);
  });
  run("validate_softmax_and_softmax_dim", [] {
    REQUIRE(Softmax::validate({})->message == "Invalid operation: Softmax - Empty tensor not supported");
    REQUIRE(!Softmax::validate({5}));
    REQUIRE(validate_softmax_dim({2, 3}, 2)->message ==
            "Invalid operation: softmax_dim - Axis 2 out of bounds for shape [2, 3]");
    REQUIRE(!validate_softmax_dim({2, 3}, 1));
  });
  run("validate_attention", [] {  // attention/tests.rs:31-47
    REQUIRE(Attention::validate({1, 1, 4, 8}, {1, 1, 2, 8}, {1, 1, 4, 8})->kind == ErrorKind::ShapeMismatch);
    REQUIRE(Attention::validate({1, 4, 8}, {1, 1, 4, 8}, {1, 1, 4, 8})->kind == ErrorKind::InvalidOperation);
    REQUIRE(!Attention::validate({1, 2, 4, 8}, {1, 2, 6, 8}, {1, 2, 6, 8}));  // cross-attention
    REQUIRE(ScaledDotProductAttention::validate({4, 8}, {4, 8}, {4, 8})->kind == ErrorKind::InvalidInput);
    REQUIRE(CausalAttention::validate({1, 1, 4, 8}, {1, 1, 4, 8}, {1, 1, 4, 4})->kind == ErrorKind::ShapeMismatch);
    REQUIRE(FlashAttention::validate({4, 8}, {4, 4}, {4, 8})->kind == ErrorKind::InvalidOperation);
    REQUIRE(FlashAttention::validate({1, 4, 8}, {1, 4, 8}, {1, 4, 8})->message.find("2D") != std::string::npos);
  });
  run("validate_gqa_and_mha", [] {  // grouped_query_attention/mod.rs:84-147, mha/mod.rs:62-126
    REQUIRE(GroupedQueryAttention::validate({1, 8, 4}, {1, 2, 4, 4}, {1, 2, 4, 4})->kind == ErrorKind::InvalidInput);
    REQUIRE(GroupedQueryAttention::validate({1, 8, 4, 4}, {1, 2, 5, 4}, {1, 2, 5, 4})->kind ==
            ErrorKind::ShapeMismatch);
    REQUIRE(GroupedQueryAttention::validate({1, 8, 4, 4}, {1, 3, 4, 4}, {1, 3, 4, 4})->message ==
            "Invalid input: num_q_heads (8) must be divisible by num_kv_heads (3)");
    REQUIRE(!GroupedQueryAttention::validate({1, 8, 4, 4}, {1, 2, 4, 4}, {1, 2, 4, 4}));
    const std::vector<size_t> x{2, 8, 64}, w{64, 64};
    const std::array<std::vector<size_t>, 4> ws{w, w, w, w};
    REQUIRE(MultiHeadAttention::validate({16, 64}, x, x, ws, 8)->kind == ErrorKind::ShapeMismatch);
    REQUIRE(MultiHeadAttention::validate(x, {2, 16, 64}, {2, 8, 64}, ws, 8)->kind == ErrorKind::ShapeMismatch);
    REQUIRE(MultiHeadAttention::validate(x, x, x, {w, w, std::vector<size_t>{64, 32}, w}, 8)->kind ==
            ErrorKind::ShapeMismatch);
    REQUIRE(MultiHeadAttention::validate(x, x, x, ws, 7)->message ==
            "Invalid operation: multi_head_attention - d_model (64) must be divisible by num_heads (7)");
    REQUIRE(!MultiHeadAttention::validate(x, {2, 16, 64}, {2, 16, 64}, ws, 8));  // cross-attention
  });
  run("validate_layer_norm", [] {  // ops/layer_norm_wgsl.rs:160-165
    REQUIRE(LayerNorm::validate({})->message == "Invalid operation: LayerNorm - Empty tensor not supported");
    REQUIRE(!LayerNorm::validate({3}));
    REQUIRE(!LayerNorm::validate({2, 3, 4}));
  });
  run("validate_fused_mlp", [] {  // nn/fused_mlp.rs:44-97 (runs before any device use)
    auto r = nn::fused_mlp(Tensor::null_for_tests({4, 8}), {}, {});
    REQUIRE(r.is_err() && r.error().message == "Invalid input: fused_mlp: at least one layer required");
    auto r2 = nn::fused_mlp(Tensor::null_for_tests({4, 8, 1}), {Tensor::null_for_tests({16, 8})},
                            {Tensor::null_for_tests({16})});
    REQUIRE(r2.is_err() && r2.error().message == "Invalid input: fused_mlp: input must be 2D, got [4, 8, 1]");
    auto r3 = nn::fused_mlp(Tensor::null_for_tests({4, 8}), {Tensor::null_for_tests({5, 7})},
                            {Tensor::null_for_tests({5})});
    REQUIRE(r3.is_err() && r3.error().message == "Invalid input: fused_mlp: weight[0] shape [5, 7] incompatible");
    auto r4 = nn::fused_mlp(Tensor::null_for_tests({4, 8}), {Tensor::null_for_tests({16, 8})},
                            {Tensor::null_for_tests({8})});
    REQUIRE(r4.is_err() && r4.error().message == "Invalid input: fused_mlp: bias[0] shape mismatch");
  });
  run("status_to_error_mapping", [] {
    REQUIRE(BarracudaError::from_status(BCH_E_OOM, "x", "op").kind == ErrorKind::OutOfMemory);
    REQUIRE(BarracudaError::from_status(BCH_E_SHAPE, "x", "matmul").kind == ErrorKind::InvalidOperation);
    REQUIRE(has_shape_words(BarracudaError::from_status(BCH_E_SHAPE, "x", "matmul").message));
    REQUIRE(BarracudaError::from_status(BCH_E_NO_DEVICE, "x", "op").kind == ErrorKind::DeviceNotAvailable);
    REQUIRE(BarracudaError::from_status(BCH_E_NO_DEVICE, "no GPU", "op").message ==
            "Device not available: hip - no GPU");  // error.rs:92-99 #[error] form
    REQUIRE(BarracudaError::from_status(BCH_E_UNSUPPORTED, "x", "op").kind == ErrorKind::UnsupportedOperation);
    REQUIRE(BarracudaError::from_status(BCH_E_LAUNCH, "x", "op").kind == ErrorKind::ExecutionError);
    REQUIRE(BarracudaError::from_status(BCH_E_INVALID, "x", "op").kind == ErrorKind::InvalidInput);
    REQUIRE(BarracudaError::from_status(BCH_E_MODULE, "x", "op").kind == ErrorKind::Device);
    REQUIRE(BarracudaError::from_status(BCH_E_DEVICE, "x", "op").kind == ErrorKind::Device);
    const auto lost = BarracudaError::from_status(BCH_E_DEVICE_LOST, "fault", "op");
    REQUIRE(lost.kind == ErrorKind::DeviceLost && lost.message == "GPU device lost: fault");  // error.rs:59
    REQUIRE(std::string(bch_status_string(BCH_E_DEVICE_LOST)) == "device lost");
    int flag = 7;
    REQUIRE(bch_ctx_is_lost(nullptr, &flag) == BCH_E_INVALID);
  });
  run("attention_dims_and_session_errors", [] {  // session/mod.rs:78-98, error.rs:436-445
    AttentionDims d{4, 32, 2048, 128};
    REQUIRE(d.total_elements() == 4ull * 32 * 2048 * 128);
    auto u = d.as_u32().unwrap();
    REQUIRE(u[0] == 4 && u[1] == 2048 && u[2] == 32 && u[3] == 128);  // (batch, seq, heads, dim)
    auto big = AttentionDims{1, 1, (size_t)UINT32_MAX + 1, 1}.as_u32();
    REQUIRE(big.is_err() && big.error().kind == ErrorKind::CastOverflow);
    REQUIRE(big.error().message == "Cast overflow: usize → u32 (4294967296)");
    REQUIRE(BarracudaError::invalid_shape({1, 2, 3}, {1, 2}).message == "Invalid shape: expected [1, 2, 3], got [1, 2]");
  });
}

// ---------------------------------------------------------------- GPU tests
void gpu_tests() {
  // ops/matmul.rs tests
  run("test_matmul_basic", [] {  // matmul.rs:264-290
    std::vector<float> a = {1, 2, 3, 4, 5, 6}, b = {1, 2, 3, 4, 5, 6};
    auto r = T(a, {2, 3}).matmul(T(b, {3, 2})).unwrap();
    REQUIRE((r.shape() == std::vector<size_t>{2, 2}));
    auto out = r.to_vec().unwrap(), exp = matmul_cpu(a, b, 2, 3, 2);
    for (size_t i = 0; i < out.size(); ++i) REQUIRE(std::fabs(out[i] - exp[i]) < 1e-5f);
  });
  run("test_matmul_edge_cases", [] {  // matmul.rs:292-336: identity, zeros
    auto r = T({1, 0, 0, 1}, {2, 2}).matmul(T({5, 6, 7, 8}, {2, 2})).unwrap().to_vec().unwrap();
    std::vector<float> e = {5, 6, 7, 8};
    for (size_t i = 0; i < 4; ++i) REQUIRE(std::fabs(r[i] - e[i]) < 1e-5f);
    auto z = T({0, 0, 0, 0}, {2, 2}).matmul(T({1, 2, 3, 4}, {2, 2})).unwrap().to_vec().unwrap();
    for (float v : z) REQUIRE(std::fabs(v) < 1e-6f);
  });
  run("test_matmul_single_element", [] {  // matmul.rs:338-356
    auto r = T({5}, {1, 1}).matmul(T({3}, {1, 1})).unwrap().to_vec().unwrap();
    REQUIRE(std::fabs(r[0] - 15.0f) < 1e-5f);
  });
  run("test_matmul_rectangular", [] {  // matmul.rs:358-377
    std::vector<float> a = {1, 2, 3, 4, 5, 6, 7, 8}, b = {1, 0, 0, 0, 1, 0};
    auto r = T(a, {4, 2}).matmul(T(b, {2, 3})).unwrap();
    REQUIRE((r.shape() == std::vector<size_t>{4, 3}));
    auto out = r.to_vec().unwrap(), exp = matmul_cpu(a, b, 4, 2, 3);
    for (size_t i = 0; i < out.size(); ++i) REQUIRE(std::fabs(out[i] - exp[i]) < 1e-5f);
  });
  run("test_matmul_large_tensor", [] {  // matmul.rs:379-409 (bound widened to 1e-6 relative at |C| ~ 7e3)
    const size_t m = 64, k = 32, n = 64;
    std::vector<float> a(m * k), b(k * n);
    for (size_t i = 0; i < a.size(); ++i) a[i] = (float)i * 0.01f;
    for (size_t i = 0; i < b.size(); ++i) b[i] = (float)i * 0.01f;
    auto out = T(a, {m, k}).matmul(T(b, {k, n})).unwrap().to_vec().unwrap();
    auto exp = matmul_cpu(a, b, m, k, n);
    for (size_t i = 0; i < out.size(); ++i)
      REQUIRE(std::fabs(out[i] - exp[i]) < std::fmax(1e-3f, 2e-6f * std::fabs(exp[i])));
  });
  run("test_matmul_precision", [] {  // matmul.rs:411-443
    std::vector<float> a = {1.234f, 2.345f, 3.456f, 4.567f, 5.678f, 6.789f};
    std::vector<float> b = {0.111f, 0.222f, 0.333f, 0.444f, 0.555f, 0.666f};
    auto out = T(a, {2, 3}).matmul_ref(T(b, {3, 2})).unwrap().to_vec().unwrap();
    auto exp = matmul_cpu(a, b, 2, 3, 2);
    for (size_t i = 0; i < 4; ++i) REQUIRE(std::fabs(out[i] - exp[i]) < 1e-5f);
  });
  run("test_matmul_tiled_and_decode_shape", [] {  // matmul_tiled.rs; skinny path m = 1
    std::vector<float> a(300), b(300 * 64);
    for (size_t i = 0; i < a.size(); ++i) a[i] = (float)((int)(i % 7) - 3);
    for (size_t i = 0; i < b.size(); ++i) b[i] = (float)((int)(i % 5) - 2);
    auto out = T(a, {1, 300}).matmul_tiled(T(b, {300, 64})).unwrap().to_vec().unwrap();
    auto exp = matmul_cpu(a, b, 1, 300, 64);
    for (size_t i = 0; i < out.size(); ++i) REQUIRE(out[i] == exp[i]);  // integers: exact
  });
  // ops/batch_matmul.rs:172-199
  run("test_batch_matmul_basic", [] {
    std::vector<float> a = {1, 2, 3, 4, 5, 6, 1, 1, 1, 2, 2, 2};
    std::vector<float> b = {1, 0, 0, 1, 1, 1, 2, 0, 0, 2, 1, 1};
    auto r = T(a, {2, 2, 3}).batch_matmul(T(b, {2, 3, 2})).unwrap();
    REQUIRE((r.shape() == std::vector<size_t>{2, 2, 2}));
    auto out = r.to_vec().unwrap();
    std::vector<float> e = {4, 5, 10, 11, 3, 3, 6, 6};
    for (size_t i = 0; i < 8; ++i) REQUIRE(out[i] == e[i]);
  });
  // ops/softmax.rs tests (global softmax)
  run("test_softmax_basic", [] {  // softmax.rs:151-166
    auto r = T({1, 2, 3}, {3}).softmax().unwrap().to_vec().unwrap();
    float sum = r[0] + r[1] + r[2];
    for (float v : r) REQUIRE(v > 0.0f && v < 1.0f);
    REQUIRE(std::fabs(sum - 1.0f) < 1e-5f);
    REQUIRE(r[2] > r[1] && r[1] > r[0]);
  });
  run("test_softmax_small_and_large_values", [] {  // softmax.rs:168-191
    auto s = T({1e-6f, 2e-6f, 3e-6f}, {3}).softmax().unwrap().to_vec().unwrap();
    REQUIRE(std::fabs(s[0] + s[1] + s[2] - 1.0f) < 1e-5f);
    auto l = T({100, 200, 300}, {3}).softmax().unwrap().to_vec().unwrap();
    REQUIRE(std::fabs(l[0] + l[1] + l[2] - 1.0f) < 1e-5f && l[2] > 0.99f);
  });
  run("test_softmax_large_input", [] {  // softmax.rs:193-206
    std::vector<float> x(1000);
    for (size_t i = 0; i < x.size(); ++i) x[i] = (float)i / 10.0f;
    auto r = T(x, {1000}).softmax().unwrap().to_vec().unwrap();
    double sum = 0;
    for (float v : r) sum += v;
    REQUIRE(std::fabs(sum - 1.0) < 1e-4);
  });
  run("test_softmax_vs_cpu", [] {  // softmax.rs:208-233
    std::vector<float> x = {1, 2, 3, 4, 5};
    auto r = T(x, {5}).softmax().unwrap().to_vec().unwrap();
    float mx = 5, sum = 0;
    std::vector<float> e(5);
    for (int i = 0; i < 5; ++i) sum += e[i] = std::exp(x[i] - mx);
    for (int i = 0; i < 5; ++i) REQUIRE(std::fabs(r[i] - e[i] / sum) < 1e-5f);
  });
  // ops/tensor_axis_ops.rs tests (softmax_dim)
  run("test_softmax_dim_rows_and_columns", [] {  // tensor_axis_ops.rs:158-200
    auto r = T({1, 2, 3, 4, 5, 6}, {2, 3}).softmax_dim(1).unwrap();
    REQUIRE((r.shape() == std::vector<size_t>{2, 3}));
    auto v = r.to_vec().unwrap();
    REQUIRE(std::fabs(v[0] + v[1] + v[2] - 1.0f) < 1e-5f && std::fabs(v[3] + v[4] + v[5] - 1.0f) < 1e-5f);
    auto c = T({1, 4, 2, 5, 3, 6}, {3, 2}).softmax_dim(0).unwrap().to_vec().unwrap();
    REQUIRE(std::fabs(c[0] + c[2] + c[4] - 1.0f) < 1e-5f && std::fabs(c[1] + c[3] + c[5] - 1.0f) < 1e-5f);
    auto one = T({1, 2, 3}, {3, 1}).softmax_dim(1).unwrap().to_vec().unwrap();
    REQUIRE((one == std::vector<float>{1, 1, 1}));
    REQUIRE(T({1, 2, 3}, {3}).softmax_dim(1).is_err());
  });
  // ops/attention/tests.rs
  run("test_attention_basic", [] {  // attention/tests.rs:8-29
    auto q = T(std::vector<float>(32, 1.0f), {1, 1, 4, 8});
    auto k = T(std::vector<float>(32, 1.0f), {1, 1, 4, 8});
    auto v = T(std::vector<float>(32, 2.0f), {1, 1, 4, 8});
    auto o = q.attention(k, v).unwrap();
    REQUIRE((o.shape() == std::vector<size_t>{1, 1, 4, 8}));
    for (float x : o.to_vec().unwrap()) REQUIRE(std::fabs(x - 2.0f) < 0.1f);
  });
  run("test_attention_shape_validation", [] {  // attention/tests.rs:31-47
    auto q = T(std::vector<float>(32, 1.0f), {1, 1, 4, 8});
    auto k = T(std::vector<float>(16, 1.0f), {1, 1, 2, 8});
    auto v = T(std::vector<float>(32, 1.0f), {1, 1, 4, 8});
    REQUIRE(q.attention(k, v).is_err());
  });
  run("test_attention_multi_head", [] {  // attention/tests.rs:49-66
    const size_t size = 2 * 4 * 8 * 16;
    auto q = T(std::vector<float>(size, 0.5f), {2, 4, 8, 16});
    auto v = T(std::vector<float>(size, 1.0f), {2, 4, 8, 16});
    auto out = q.attention(q, v).unwrap().to_vec().unwrap();
    REQUIRE(out.size() == size);
    for (float x : out) REQUIRE(std::isfinite(x) && std::fabs(x - 1.0f) < 1e-6f);
  });
  run("test_sdpa_and_causal", [] {  // sdpa + causal: row 0 of causal attends to key 0 only
    const size_t S = 5, D = 3;
    std::vector<float> q(S * D, 0.0f), k(S * D, 1.0f), v(S * D);
    for (size_t i = 0; i < v.size(); ++i) v[i] = (float)i;
    auto tq = T(q, {1, 1, S, D}), tk = T(k, {1, 1, S, D}), tv = T(v, {1, 1, S, D});
    auto c = tq.causal_attention(tk, tv).unwrap().to_vec().unwrap();
    for (size_t i = 0; i < S; ++i)  // equal scores: row i = mean of V[0..=i]
      for (size_t d = 0; d < D; ++d) {
        float mean = 0;
        for (size_t j = 0; j <= i; ++j) mean += v[j * D + d];
        REQUIRE(std::fabs(c[i * D + d] - mean / (float)(i + 1)) < 1e-5f);
      }
    auto s = tq.scaled_dot_product_attention(tk, tv).unwrap().to_vec().unwrap();
    for (size_t d = 0; d < D; ++d) {
      float mean = 0;
      for (size_t j = 0; j < S; ++j) mean += v[j * D + d];
      REQUIRE(std::fabs(s[d] - mean / (float)S) < 1e-5f);
    }
  });
  run("test_flash_attention_single_head", [] {  // flash_attention.rs:152-185
    auto q = T(std::vector<float>(64, 0.3f), {16, 4});
    auto v = T(std::vector<float>(64, 2.0f), {16, 4});
    auto out = FlashAttention{q, q, v, 1}.execute().unwrap().to_vec().unwrap();
    for (float x : out) REQUIRE(std::fabs(x - 2.0f) < 1e-5f);
  });
  // crates/barracuda/tests/fault_injection.rs:29-60
  run("test_grouped_query_attention_basic", [] {  // grouped_query_attention/tests.rs:21-38
    auto q = T(std::vector<float>(8 * 16, 0.5f), {1, 8, 4, 4});
    auto kv = T(std::vector<float>(2 * 16, 0.5f), {1, 2, 4, 4});
    auto out = q.grouped_query_attention(kv, kv).unwrap();
    REQUIRE(out.shape() == (std::vector<size_t>{1, 8, 4, 4}));
    for (float x : out.to_vec().unwrap()) REQUIRE(std::fabs(x - 0.5f) <= 1e-6f);
  });
  run("test_mha_basic_and_cross_attention", [] {  // mha/tests.rs:9-56, :98-149
    // q = k = 0.5, v = 1, all weights 0.01, d_model 64, 8 heads: 0.64 per head, out = 0.64 * 0.01 * 64
    for (size_t skv : {8, 16}) {
      auto q = T(std::vector<float>(2 * 8 * 64, 0.5f), {2, 8, 64});
      auto k = T(std::vector<float>(2 * skv * 64, 0.5f), {2, skv, 64});
      auto v = T(std::vector<float>(2 * skv * 64, 1.0f), {2, skv, 64});
      auto w = T(std::vector<float>(64 * 64, 0.01f), {64, 64});
      auto out = q.multi_head_attention(k, v, w, w, w, w, 8).unwrap();
      REQUIRE(out.shape() == (std::vector<size_t>{2, 8, 64}));
      const double w64 = (double)0.01f, want = 64 * w64 * 64 * w64;
      for (float x : out.to_vec().unwrap()) REQUIRE(std::fabs(x - want) <= 1e-5 * want);
    }
    auto q = T(std::vector<float>(2 * 8 * 64, 0.5f), {2, 8, 64});
    auto w = T(std::vector<float>(64 * 64, 0.01f), {64, 64});
    REQUIRE(q.multi_head_attention(q, q, w, w, w, w, 7).is_err());  // mha/tests.rs:59-96
  });
  run("test_fused_mlp_two_layers", [] {  // nn/fused_mlp.rs: linear + relu per layer, W [out, in]
    const size_t batch = 3, d0 = 4, d1 = 5, d2 = 2;
    std::vector<float> x(batch * d0), w0(d1 * d0), b0(d1), w1(d2 * d1), b1(d2);
    for (size_t i = 0; i < x.size(); ++i) x[i] = (float)((int)(i % 7) - 3);
    for (size_t i = 0; i < w0.size(); ++i) w0[i] = (float)((int)(i % 5) - 2);
    for (size_t i = 0; i < w1.size(); ++i) w1[i] = (float)((int)(i % 3) - 1);
    for (size_t i = 0; i < d1; ++i) b0[i] = (float)i - 2.0f;
    for (size_t i = 0; i < d2; ++i) b1[i] = 0.5f;
    auto out = nn::fused_mlp(T(x, {batch, d0}), {T(w0, {d1, d0}), T(w1, {d2, d1})}, {T(b0, {d1}), T(b1, {d2})},
                             nn::Activation::ReLU)
                   .unwrap();
    REQUIRE(out.shape() == (std::vector<size_t>{batch, d2}));
    // integer-valued: exact
    std::vector<float> h(batch * d1), y(batch * d2);
    for (size_t b = 0; b < batch; ++b) {
      for (size_t o = 0; o < d1; ++o) {
        float s = 0;
        for (size_t i = 0; i < d0; ++i) s += x[b * d0 + i] * w0[o * d0 + i];
        h[b * d1 + o] = std::fmax(s + b0[o], 0.0f);
      }
      for (size_t o = 0; o < d2; ++o) {
        float s = 0;
        for (size_t i = 0; i < d1; ++i) s += h[b * d1 + i] * w1[o * d1 + i];
        y[b * d2 + o] = std::fmax(s + b1[o], 0.0f);
      }
    }
    REQUIRE(out.to_vec().unwrap() == y);
  });
  run("test_relu_gelu_layer_norm", [] {  // ops/relu.rs, ops/gelu_wgsl.rs, ops/layer_norm_wgsl.rs:166-192
    std::vector<float> x(3 * 1000);
    for (size_t i = 0; i < x.size(); ++i) x[i] = 0.01f * (float)((int)(i * 37 % 1201) - 600);
    auto t = T(x, {3, 1000});
    // relu is one IEEE max per element: exact
    auto r = t.relu().unwrap();
    REQUIRE(r.shape() == t.shape());
    auto rv = r.to_vec().unwrap();
    for (size_t i = 0; i < x.size(); ++i) REQUIRE(rv[i] == std::fmax(x[i], 0.0f));
    // gelu: the tanh form in double, |err| <= 1e-4 max(|ref|, 1)
    auto gv = t.gelu_wgsl().unwrap().to_vec().unwrap();
    for (size_t i = 0; i < x.size(); ++i) {
      const double v = x[i], ref = 0.5 * v * (1.0 + std::tanh(0.7978845608028654 * (v + 0.044715 * v * v * v)));
      REQUIRE(std::fabs(gv[i] - ref) <= 1e-4 * std::fmax(std::fabs(ref), 1.0));
    }
    REQUIRE(T({0.0f}, {1}).gelu_wgsl().unwrap().to_vec().unwrap()[0] == 0.0f);
    // layer norm: [1, 2, 3, 4]'s closed form, zero row means, constant rows exactly 0
    auto y = T({1, 2, 3, 4}, {1, 4}).layer_norm_wgsl(1e-5f).unwrap().to_vec().unwrap();
    for (int i = 0; i < 4; ++i) REQUIRE(std::fabs(y[i] - (i + 1 - 2.5) / std::sqrt(1.25 + 1e-5)) < 1e-6);
    auto lv = t.layer_norm_wgsl(1e-5f).unwrap().to_vec().unwrap();
    for (size_t row = 0; row < 3; ++row) {
      double mean = 0, var = 0;
      for (size_t c = 0; c < 1000; ++c) mean += x[row * 1000 + c];
      mean /= 1000;
      for (size_t c = 0; c < 1000; ++c) var += (x[row * 1000 + c] - mean) * (x[row * 1000 + c] - mean);
      var /= 1000;
      for (size_t c = 0; c < 1000; ++c) {
        const double ref = (x[row * 1000 + c] - mean) / std::sqrt(var + 1e-5);
        REQUIRE(std::fabs(lv[row * 1000 + c] - ref) <= 1e-4 * std::fmax(std::fabs(ref), 1.0));
      }
    }
    auto z = T(std::vector<float>(2 * 64, 3.0f), {2, 64}).layer_norm_wgsl(1e-5f).unwrap().to_vec().unwrap();
    for (float v : z) REQUIRE(v == 0.0f);
  });
  run("test_fused_mlp_gelu", [] {  // GELU in the GEMM epilogue, W [out, in]
    const size_t batch = 5, d0 = 64, d1 = 48;
    std::vector<float> x(batch * d0), w(d1 * d0), b(d1);
    for (size_t i = 0; i < x.size(); ++i) x[i] = 0.125f * (float)((int)(i % 9) - 4);
    for (size_t i = 0; i < w.size(); ++i) w[i] = 0.0625f * (float)((int)(i % 7) - 3);
    for (size_t i = 0; i < d1; ++i) b[i] = 0.25f * (float)((int)i % 5 - 2);
    auto out = nn::fused_mlp(T(x, {batch, d0}), {T(w, {d1, d0})}, {T(b, {d1})}, nn::Activation::GELU).unwrap();
    REQUIRE(out.shape() == (std::vector<size_t>{batch, d1}));
    auto got = out.to_vec().unwrap();
    for (size_t r = 0; r < batch; ++r)
      for (size_t o = 0; o < d1; ++o) {
        double s = b[o];
        for (size_t i = 0; i < d0; ++i) s += (double)x[r * d0 + i] * w[o * d0 + i];
        const double ref = 0.5 * s * (1.0 + std::tanh(0.7978845608028654 * (s + 0.044715 * s * s * s)));
        REQUIRE(std::fabs(got[r * d1 + o] - ref) <= 1e-4 * std::fmax(std::fabs(ref), 1.0));
      }
  });
  run("test_gemm_f64_basic_transpose_batched", [] {  // ops/linalg/gemm_f64.rs tests
    const std::vector<double> want{19, 22, 43, 50};
    REQUIRE(GemmF64::execute(g_dev, {1, 2, 3, 4}, {5, 6, 7, 8}, 2, 2, 2, 1).unwrap() == want);
    REQUIRE(GemmF64::execute_gemm_ex(g_dev, {1, 3, 2, 4}, {5, 6, 7, 8}, 2, 2, 2, 1, 1.0, 0.0, true, false).unwrap() ==
            want);
    REQUIRE(GemmF64::execute_gemm_ex(g_dev, {1, 2, 3, 4}, {5, 7, 6, 8}, 2, 2, 2, 1, 1.0, 0.0, false, true).unwrap() ==
            want);
    std::vector<double> a{1, 0, 0, 0, 1, 0, 0, 0, 1, 2, 0, 0, 0, 2, 0, 0, 0, 2}, b;
    for (int r = 0; r < 2; ++r)
      for (int i = 1; i <= 9; ++i) b.push_back(i);
    auto c = GemmF64::execute(g_dev, a, b, 3, 3, 3, 2).unwrap();
    REQUIRE(c[0] == 1.0 && c[4] == 5.0 && c[9] == 2.0 && c[13] == 10.0);
    REQUIRE(GemmF64::execute(g_dev, {1, 2, 3}, {1, 2, 3, 4}, 2, 2, 2, 1).error().message ==
            "Invalid input: A: expected 4 elements, got 3");
    auto cached = GemmCachedF64::create(g_dev, {5, 6, 7, 8, 9, 10}, 2, 3, 1).unwrap();
    REQUIRE(cached.multiply({1, 2}, 1).unwrap() == (std::vector<double>{21, 24, 27}));  // [1 2] [[5 6 7] [8 9 10]]
  });
  run("test_fault_injection_shape_mismatch", [] {
    auto r = T({1, 2, 3, 4, 5, 6}, {2, 3}).matmul(T({1, 2, 3, 4, 5, 6, 7, 8}, {4, 2}));
    REQUIRE(r.is_err() && has_shape_words(r.error().message));
    // the device stays usable after the error
    auto ok = T({1, 1, 1, 1, 1, 1}, {2, 3}).matmul(T({1, 1, 1, 1, 1, 1}, {3, 2})).unwrap().to_vec().unwrap();
    for (float x : ok) REQUIRE(x == 3.0f);
  });
  run("test_tensor_from_data_size_mismatch", [] {
    auto r = Tensor::from_data({1, 2, 3}, {2, 2}, g_dev);
    REQUIRE(r.is_err() && r.error().kind == ErrorKind::ShapeMismatch);
  });

  // session/mod.rs tests
  run("test_session_matmul_2x2", [] {  // session/mod.rs:678-694
    TensorSession s(g_dev);
    auto a = s.tensor_with_shape({1, 2, 3, 4}, {2, 2}).unwrap();
    auto b = s.tensor_with_shape({5, 6, 7, 8}, {2, 2}).unwrap();
    auto c = s.matmul(a, b).unwrap();
    REQUIRE((c.shape() == std::vector<size_t>{2, 2}));
    s.run().unwrap();
    auto r = c.to_vec().unwrap();
    const float e[4] = {19, 22, 43, 50};
    for (int i = 0; i < 4; ++i) REQUIRE(std::fabs(r[i] - e[i]) < 0.01f);
  });
  run("test_session_reset_and_reuse", [] {  // session/mod.rs:710-723, with matmul for add
    TensorSession s(g_dev);
    auto a = s.tensor_with_shape({1, 2}, {1, 2}).unwrap();
    auto b = s.tensor_with_shape({3, 4}, {2, 1}).unwrap();
    auto c = s.matmul(a, b).unwrap();
    REQUIRE(c.to_vec().unwrap()[0] == 0.0f);  // allocated, not yet computed
    s.run().unwrap();
    REQUIRE(c.to_vec().unwrap()[0] == 11.0f);
    s.reset();
    REQUIRE(s.num_ops() == 0 && !s.executed());
    auto z = s.softmax(s.tensor({0, 0, 0, 0}).unwrap()).unwrap();
    s.run().unwrap();
    for (float x : z.to_vec().unwrap()) REQUIRE(x == 0.25f);
    REQUIRE(c.to_tensor().unwrap().to_vec().unwrap()[0] == 11.0f);
  });
  run("test_session_ops_match_tensor_ops", [] {
    // non-square matmul, softmax over > 256 elements, attention: the session
    // runs the same kernels as the Tensor ops, so results are bit-identical
    const size_t m = 37, k = 300, n = 129;
    std::vector<float> a(m * k), b(k * n);
    for (size_t i = 0; i < a.size(); ++i) a[i] = (float)((i * 7919) % 23) / 11.0f - 1.0f;
    for (size_t i = 0; i < b.size(); ++i) b[i] = (float)((i * 104729) % 19) / 9.0f - 1.0f;
    TensorSession s(g_dev);
    auto sc = s.matmul(s.tensor_with_shape(a, {m, k}).unwrap(), s.tensor_with_shape(b, {k, n}).unwrap()).unwrap();
    auto sp = s.softmax(sc).unwrap();
    const size_t B = 2, H = 3, S = 40, D = 16;
    std::vector<float> q(B * H * S * D);
    for (size_t i = 0; i < q.size(); ++i) q[i] = (float)((i * 31) % 17) / 8.0f - 1.0f;
    auto tq = s.tensor(q).unwrap();
    auto so = s.attention(tq, tq, tq, AttentionDims{B, H, S, D}).unwrap();
    REQUIRE(s.num_ops() == 3);
    REQUIRE((so.shape() == std::vector<size_t>{B, H, S, D}));
    s.run().unwrap();
    auto c = T(a, {m, k}).matmul(T(b, {k, n})).unwrap();
    REQUIRE(sc.to_vec().unwrap() == c.to_vec().unwrap());
    REQUIRE(sp.to_vec().unwrap() == c.softmax().unwrap().to_vec().unwrap());
    auto qt = T(q, {B, H, S, D});
    REQUIRE(so.to_vec().unwrap() == qt.attention(qt, qt).unwrap().to_vec().unwrap());
    auto ref = matmul_cpu(a, b, m, k, n);
    auto got = sc.to_vec().unwrap();
    for (size_t i = 0; i < ref.size(); ++i) REQUIRE(std::fabs(got[i] - ref[i]) <= 1e-4f * std::fmax(1.0f, std::fabs(ref[i])));
  });
  run("test_session_head_split_concat", [] {  // session/mod.rs:423-480 with the recipe of :481-518
    const size_t B = 2, S = 5, H = 3, D = 6;
    std::vector<float> x(B * S * H * D);
    for (size_t i = 0; i < x.size(); ++i) x[i] = (float)i;  // exact in f32
    TensorSession s(g_dev);
    AttentionDims dims{B, H, S, D};
    auto in = s.tensor_with_shape(x, {B, S, H * D}).unwrap();
    auto split = s.head_split(in, dims).unwrap();
    REQUIRE((split.shape() == std::vector<size_t>{B, H, S, D}));
    auto att = s.attention(split, split, split, dims).unwrap();
    auto back = s.head_concat(split, dims).unwrap();
    auto cat = s.head_concat(att, dims).unwrap();
    REQUIRE((back.shape() == std::vector<size_t>{B, S, H * D}));
    REQUIRE(s.num_ops() == 4);
    s.run().unwrap();
    auto sp = split.to_vec().unwrap();
    for (size_t b = 0; b < B; ++b)
      for (size_t h = 0; h < H; ++h)
        for (size_t t = 0; t < S; ++t)
          for (size_t d = 0; d < D; ++d)  // head_split_f64.wgsl: out[b][h][s][d] = in[b][s][h*D + d]
            REQUIRE(sp[((b * H + h) * S + t) * D + d] == x[(b * S + t) * H * D + h * D + d]);
    REQUIRE(back.to_vec().unwrap() == x);  // head_concat inverts head_split
    // the concat of attention output equals attention on the Tensor API then the same permutation
    auto ref = T(sp, {B, H, S, D}).attention(T(sp, {B, H, S, D}), T(sp, {B, H, S, D})).unwrap().to_vec().unwrap();
    auto got = cat.to_vec().unwrap();
    for (size_t b = 0; b < B; ++b)
      for (size_t h = 0; h < H; ++h)
        for (size_t t = 0; t < S; ++t)
          for (size_t d = 0; d < D; ++d)
            REQUIRE(got[(b * S + t) * H * D + h * D + d] == ref[((b * H + h) * S + t) * D + d]);
    auto bad = s.tensor(std::vector<float>(7)).unwrap();
    auto e = s.head_split(bad, dims);
    REQUIRE(e.is_err() && e.error().message == "Invalid input: head_split: input len 7 ≠ B×S×H×D=180");
    e = s.head_concat(bad, dims);
    REQUIRE(e.is_err() && e.error().message == "Invalid input: head_concat: input len 7 ≠ B×H×S×D=180");
  });
  run("test_session_validation", [] {
    TensorSession s(g_dev);
    auto r = s.tensor_with_shape({0, 0, 0, 0, 0}, {2, 3});
    REQUIRE(r.is_err() && r.error().message == "Invalid shape: expected [2, 3], got [5]");
    auto a3 = s.tensor_with_shape(std::vector<float>(8), {2, 2, 2}).unwrap();
    auto a2 = s.tensor_with_shape(std::vector<float>(6), {2, 3}).unwrap();
    auto b2 = s.tensor_with_shape(std::vector<float>(8), {2, 4}).unwrap();
    REQUIRE(s.matmul(a3, b2).error().kind == ErrorKind::InvalidShape);
    REQUIRE(s.matmul(a2, b2).error().message == "Shape mismatch: expected [2, 3], got [2, 4]");
    auto q = s.tensor(std::vector<float>(16)).unwrap();
    auto bad = s.tensor(std::vector<float>(15)).unwrap();
    auto e = s.attention(q, bad, q, AttentionDims{1, 2, 4, 2});
    REQUIRE(e.is_err() && e.error().message == "Invalid input: attention: k len 15 ≠ B×H×S×D=16");
    TensorSession other(g_dev);
    auto foreign = other.tensor({1}).unwrap();
    REQUIRE(s.softmax(foreign).error().kind == ErrorKind::InvalidInput);
    REQUIRE(s.num_ops() == 0);
    s.run().unwrap();  // nothing recorded: no-op
  });
}

}  // namespace

int main(int argc, char** argv) {
  const bool gpu = argc > 1 && std::strcmp(argv[1], "--gpu") == 0;
  cpu_tests();
  auto dr = HipDevice::create(0);
  if (!gpu) {
    // without a GPU the device constructor returns Err(Device), never aborts
    run("no_device_is_an_error_value", [&] {
      if (dr.is_ok()) return;  // a GPU is present: nothing to check here
      REQUIRE(dr.error().kind == ErrorKind::DeviceNotAvailable);
      REQUIRE(dr.error().message.find("no HIP device") != std::string::npos);
    });
  } else {
    if (dr.is_err()) {
      std::printf("FAIL device: %s\n", dr.error().message.c_str());
      return 1;
    }
    g_dev = dr.value();
    gpu_tests();
  }
  std::printf("%d passed, %d failed\n", g_pass, g_fail);
  return g_fail == 0 ? 0 : 1;
}
