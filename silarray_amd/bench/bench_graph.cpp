// Benchmarks and checks of whole sil::eval graphs through the C++ front end.
//
//   bench_graph chain   [n] [reps]            20 scalar affine nodes (x*a+b x10)
//                                             on n floats, one sil::eval
//   bench_graph encoder [B S D H F] [reps]    one transformer encoder block
//                                             (pre-norm, multi-head attention,
//                                             ReLU FFN) as one sil::eval graph
//   bench_graph encoder-dump B S D H F DIR    writes the block's inputs and
//                                             output (raw float32) to DIR for
//                                             the parity test
//   bench_graph transformer [seq d ff] [reps] the reference's single-head block
//   bench_graph mlp [batch] [reps]            the reference's linear_sigmoid MLP
//   bench_graph train [batch] [reps]          the reference's training step:
//                                             768 -> 2048 -> 768 sigmoid MLP,
//                                             forward, MSE gradient, backward,
//                                             SGD update, one sil::eval
//   bench_graph transfer [n] [reps]           host<->HBM copies of an n-float
//                                             array through its (pinned) host
//                                             mirror: upload after a host
//                                             write, download on a host read
//   bench_graph mnist [train test]            the reference's MNIST classifier
//                                             (784-50-10) and autoencoder
//                                             (784-512-256-64-256-512-784)
//                                             benchmarks: one training epoch
//                                             (batches of 100 sliced from the
//                                             resident set, SGD, one eval per
//                                             batch) and inference on the test
//                                             set; synthetic images in [0, 1)
//                                             and labels (the MNIST files are
//                                             not part of the reference)
//   bench_graph train-dump B D H DIR          one training step on seeded
//                                             inputs, written to DIR (raw
//                                             float32) for the parity test
//   bench_graph dot-dump M N K DIR            C = A.dot(B) through sil::array
//                                             on uniform[-1, 1) inputs (the
//                                             reference's SGEMM config,
//                                             bench/micro/bench_sgemm.cpp:34);
//                                             A, B and C written to DIR
//   bench_graph micro                         the reference's GPU
//                                             micro-benchmarks (bench/micro/
//                                             bench_broadcast.cpp,
//                                             bench_elementwise.cpp,
//                                             bench_nn_ops.cpp,
//                                             bench_reduction.cpp) at their
//                                             shapes: one JSON line each
//   bench_graph chain-dump n DIR              the 20-node chain of `chain` on
//                                             n uniform[-1, 1) floats, one
//                                             sil::eval; x and y written to
//                                             DIR
//
// Each timed iteration is sil::eval + wait, the reference's convention
// (bench/bench_common.h:42-68); the median of `reps` iterations is reported
// as one JSON line.  Inputs come from a SplitMix64 stream (seeded, portable)
// so the parity test can regenerate them.
#include <silarray.h>

#include <algorithm>
#include <array>
#include <stdexcept>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <string>
#include <utility>
#include <vector>

using namespace sil;

namespace {

// SplitMix64; uniform in [-1, 1) from the top 24 bits; normal by Box-Muller.
struct rng {
  uint64_t s;
  explicit rng(uint64_t seed) : s(seed) {}
  uint64_t next() {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  }
  float uniform() { return float(next() >> 40) * (2.0f / 16777216.0f) - 1.0f; }
  float normal(float std) {
    double u1 = (double(next() >> 11) + 1.0) / 9007199254740993.0;
    double u2 = double(next() >> 11) / 9007199254740992.0;
    return float(std * std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
  }
};

array<float> filled(const shape_type &shape, rng &g, float std, bool uniform = false) {
  array<float> a = array<float>::make_uninit_(shape);
  float *p = a.buffer_data();
  for (size_t i = 0; i < a.element_count(); i++) p[i] = uniform ? g.uniform() : g.normal(std);
  return a;
}

// At least two untimed runs and at least 0.2 s of them, so the GPU has left
// its idle clocks before the timed runs.
template <typename F>
double median_ms(int reps, F fn) {
  const auto w0 = std::chrono::steady_clock::now();
  for (int i = 0; i < 2 || std::chrono::steady_clock::now() - w0 < std::chrono::milliseconds(200);
       i++)
    fn();
  std::vector<double> t;
  for (int i = 0; i < reps; i++) {
    auto t0 = std::chrono::steady_clock::now();
    fn();
    auto t1 = std::chrono::steady_clock::now();
    t.push_back(std::chrono::duration<double, std::milli>(t1 - t0).count());
  }
  std::sort(t.begin(), t.end());
  return t[t.size() / 2];
}

struct encoder {
  size_t B, S, D, H, F;
  array<float> x, g1, b1, Wqkv, bqkv, Wo, bo, g2, b2, W1, c1, W2, c2;

  encoder(size_t B_, size_t S_, size_t D_, size_t H_, size_t F_, uint64_t seed)
      : B(B_), S(S_), D(D_), H(H_), F(F_) {
    rng g(seed);
    x = filled({B * S, D}, g, 1.0f);
    Wqkv = filled({D, 3 * D}, g, 0.02f);
    bqkv = filled({3 * D}, g, 0.02f);
    Wo = filled({D, D}, g, 0.02f);
    bo = filled({D}, g, 0.02f);
    W1 = filled({D, F}, g, 0.02f);
    c1 = filled({F}, g, 0.02f);
    W2 = filled({F, D}, g, 0.02f);
    c2 = filled({D}, g, 0.02f);
    g1 = ones<float>({D});
    b1 = zeros<float>({D});
    g2 = ones<float>({D});
    b2 = zeros<float>({D});
  }

  // The block as one lazy graph:
  //   h = LN1(x); [q k v] = split(h Wqkv + bqkv) into H heads of D/H
  //   attn = softmax(q k^T / sqrt(D/H)) v; r1 = x + merge(attn) Wo + bo
  //   out = r1 + relu(LN2(r1) W1 + c1) W2 + c2
  // stages() keeps the intermediate arrays (for per-stage parity checks);
  // build() drops them, so only `out` holds the graph.
  struct stages_t {
    array<float> h, qkv, merged, r1, h2, ff, out;
  };
  stages_t stages() const {
    const size_t dh = D / H;
    const float scale = 1.0f / std::sqrt(float(dh));
    stages_t st;
    st.h = x.layer_norm(g1, b1);
    st.qkv = st.h.linear(Wqkv, bqkv);                                     // [B*S, 3D]
    auto heads = st.qkv.view({B, S, 3, H, dh}).permute({2, 0, 3, 1, 4});  // [3, B, H, S, dh]
    auto q = heads.select(0, 0), k = heads.select(0, 1), v = heads.select(0, 2);
    auto scores = q.batched_dot(k.permute({0, 1, 3, 2})) * scale;         // [B, H, S, S]
    auto attn = scores.view({B * H * S, S}).softmax().view({B, H, S, S});
    auto ctx = attn.batched_dot(v);                                       // [B, H, S, dh]
    st.merged = ctx.permute({0, 2, 1, 3}).view({B * S, D});
    st.r1 = x + st.merged.linear(Wo, bo);
    st.h2 = st.r1.layer_norm(g2, b2);
    st.ff = st.h2.linear(W1, c1).relu();
    st.out = st.r1 + st.ff.linear(W2, c2);
    return st;
  }
  array<float> build() const { return stages().out; }

  double gemm_flops() const {
    const double M = double(B * S);
    return 2.0 * M * D * 3 * D + 2.0 * B * H * S * S * (D / H) * 2 + 2.0 * M * D * D +
           2.0 * M * D * F * 2;
  }
};

// The reference's single-head transformer block, written exactly as its
// composite benchmark writes it (bench/composite/bench_transformer.cpp:34-71):
// separate Q/K/V projections, scores = Q K^T * scale with K^T a transposed
// view, row softmax, one sil::eval + synchronize per iteration.
double transformer_ms(size_t seq, size_t d_model, size_t d_ff, int reps) {
  const float scale = 1.0f / std::sqrt(float(d_model));
  auto x = random({seq, d_model});
  auto Wq = random({d_model, d_model}) * scale, bq = zeros<float>({d_model});
  auto Wk = random({d_model, d_model}) * scale, bk = zeros<float>({d_model});
  auto Wv = random({d_model, d_model}) * scale, bv = zeros<float>({d_model});
  auto Wo = random({d_model, d_model}) * scale, bo = zeros<float>({d_model});
  auto W1 = random({d_model, d_ff}) * (1.0f / std::sqrt(float(d_model)));
  auto b1 = zeros<float>({d_ff});
  auto W2 = random({d_ff, d_model}) * (1.0f / std::sqrt(float(d_ff)));
  auto b2 = zeros<float>({d_model});
  auto gamma1 = ones<float>({d_model}), beta1 = zeros<float>({d_model});
  auto gamma2 = ones<float>({d_model}), beta2 = zeros<float>({d_model});
  eval(Wq, Wk, Wv, Wo, W1, W2);
  synchronize();
  return median_ms(reps, [&] {
    auto h = x.layer_norm(gamma1, beta1);
    auto Q = h.linear(Wq, bq);
    auto K = h.linear(Wk, bk);
    auto V = h.linear(Wv, bv);
    auto scores = Q.dot(K.transpose()) * scale;
    auto attn = scores.softmax();
    auto context = attn.dot(V);
    auto attn_out = context.linear(Wo, bo);
    auto r1 = x + attn_out;
    auto h2 = r1.layer_norm(gamma2, beta2);
    auto ff = h2.linear(W1, b1).relu();
    auto out = r1 + ff.linear(W2, b2);
    eval(out);
    synchronize();
  });
}

// The reference's MNIST benchmarks (bench/mnist/bench_classifier.cpp:33-73,
// 252-264; bench/mnist/bench_autoencoder.cpp:39-80, 243-256), with the same
// graphs, batch, learning rates and evaluation points, on synthetic data of
// the MNIST shapes.  Each figure is the wall time of one timed run after one
// untimed run (the reference's measure(0, fn, 0, 1) runs the epoch once to
// calibrate, then once timed).
struct mnist_result {
  double classifier_train_ms, classifier_infer_ms, autoencoder_train_ms, autoencoder_infer_ms;
  float classifier_mse_first, classifier_mse_last;
};

template <typename F>
double once_ms(F fn) {
  fn();  // untimed
  synchronize();
  const auto t0 = std::chrono::steady_clock::now();
  fn();
  synchronize();
  return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
}

mnist_result mnist_bench(size_t n_train, size_t n_test) {
  constexpr size_t D = 784, H = 50, C = 10, batch = 100;
  rng g(31);
  std::vector<float> img_train(n_train * D), img_test(n_test * D), labels(n_train);
  for (auto &v : img_train) v = 0.5f * (g.uniform() + 1.0f);
  for (auto &v : img_test) v = 0.5f * (g.uniform() + 1.0f);
  for (auto &v : labels) v = float(g.next() % C);
  mnist_result r{};
  {  // classifier training (bench_classifier.cpp:33-73)
    const float lr = 0.5f;
    auto W1 = (random({D, H}) * 2.0f - 1.0f) * (1.0f / std::sqrt(float(D)));
    auto b1 = zeros<float>({H});
    auto W2 = (random({H, C}) * 2.0f - 1.0f) * (1.0f / std::sqrt(float(H)));
    auto b2 = zeros<float>({C});
    auto two = array<float>(2.0f);
    auto inv_n = array<float>(1.0f / float(batch * C));
    auto neg_lr = array<float>(-lr);
    auto all_x = array<float>({n_train, D}, img_train.data());
    auto all_labels = array<float>({n_train}, labels.data());
    auto all_Y = all_labels.template one_hot<float>(C);
    eval(W1, W2, all_x, all_Y);
    synchronize();
    float mse_first = 0.0f, mse_last = 0.0f;
    auto epoch = [&] {
      for (size_t i = 0; i + batch <= n_train; i += batch) {
        auto x = all_x.slice(i, batch);
        auto Y = all_Y.slice(i, batch);
        auto n1 = x.linear(W1, b1);
        auto o1 = n1.sigmoid();
        auto n2 = o1.linear(W2, b2);
        auto o2 = n2.sigmoid();
        auto dout = (o2 - Y) * two * inv_n;
        dout = n2.sigmoid_backward(dout);
        auto dW2 = o1.transpose().dot(dout);
        auto db2 = dout.sum(0);
        auto dout1 = dout.dot(W2.transpose());
        dout1 = n1.sigmoid_backward(dout1);
        auto dW1 = x.transpose().dot(dout1);
        auto db1 = dout1.sum(0);
        W1 = W1 + dW1 * neg_lr;
        b1 = b1 + db1 * neg_lr;
        W2 = W2 + dW2 * neg_lr;
        b2 = b2 + db2 * neg_lr;
        eval(W1, b1, W2, b2);
      }
    };
    auto mse = [&] {  // squared error on the first batch
      auto x = all_x.slice(0, batch);
      auto d = x.linear(W1, b1).sigmoid().linear(W2, b2).sigmoid() - all_Y.slice(0, batch);
      return float((d * d).sum()) / float(batch * C);
    };
    mse_first = mse();
    r.classifier_train_ms = once_ms(epoch);
    mse_last = mse();
    r.classifier_mse_first = mse_first;
    r.classifier_mse_last = mse_last;
  }
  {  // classifier inference (bench_classifier.cpp:252-264)
    auto W1 = random({D, H});
    auto b1 = zeros<float>({H});
    auto W2 = random({H, C});
    auto b2 = zeros<float>({C});
    auto x = array<float>({n_test, D}, img_test.data());
    eval(W1, W2, x);
    synchronize();
    r.classifier_infer_ms = median_ms(20, [&] {
      auto o1 = x.linear(W1, b1).sigmoid();
      auto o2 = o1.linear(W2, b2).sigmoid();
      eval(o2);
    });
  }
  constexpr size_t L[] = {784, 512, 256, 64, 256, 512, 784};
  constexpr size_t NL = 6;
  {  // autoencoder training (bench_autoencoder.cpp:39-80)
    const float lr = 0.01f;
    array<float> W[NL], b[NL];
    for (size_t l = 0; l < NL; l++) {
      W[l] = random({L[l], L[l + 1]}) * (2.0f / std::sqrt(float(L[l])));
      b[l] = zeros<float>({L[l + 1]});
      eval(W[l]);
    }
    auto two = array<float>(2.0f);
    auto inv_n = array<float>(1.0f / float(batch * 784));
    auto neg_lr = array<float>(-lr);
    auto all_x = array<float>({n_train, 784}, img_train.data());
    eval(all_x);
    synchronize();
    r.autoencoder_train_ms = once_ms([&] {
      for (size_t i = 0; i + batch <= n_train; i += batch) {
        auto x = all_x.slice(i, batch);
        array<float> net[NL], out[NL];
        auto h = x;
        for (size_t l = 0; l < NL; l++) {
          net[l] = h.linear(W[l], b[l]);
          out[l] = net[l].sigmoid();
          h = out[l];
        }
        auto dout = (h - x) * two * inv_n;
        for (int l = int(NL) - 1; l >= 0; l--) {
          dout = net[l].sigmoid_backward(dout);
          auto &input = (l > 0) ? out[l - 1] : x;
          auto dW = input.transpose().dot(dout);
          auto db = dout.sum(0);
          if (l > 0) dout = dout.dot(W[l].transpose());
          W[l] = W[l] + dW * neg_lr;
          b[l] = b[l] + db * neg_lr;
        }
        eval(W[0], b[0], W[1], b[1], W[2], b[2], W[3], b[3], W[4], b[4], W[5], b[5]);
      }
    });
  }
  {  // autoencoder inference (bench_autoencoder.cpp:243-256)
    array<float> W[NL], b[NL];
    for (size_t l = 0; l < NL; l++) {
      W[l] = random({L[l], L[l + 1]});
      b[l] = zeros<float>({L[l + 1]});
      eval(W[l]);
    }
    auto x = array<float>({n_test, 784}, img_test.data());
    eval(x);
    synchronize();
    r.autoencoder_infer_ms = median_ms(20, [&] {
      auto h = x;
      for (size_t l = 0; l < NL; l++) h = h.linear(W[l], b[l]).sigmoid();
      eval(h);
    });
  }
  return r;
}

// The reference's MLP inference benchmark (bench/composite/bench_mlp.cpp:28-41):
// 768 -> 2048 -> sigmoid -> 768 -> sigmoid through linear_sigmoid.
double mlp_ms(size_t batch, int reps) {
  const size_t D = 768, H = 2048;
  auto x = random({batch, D});
  auto W1 = random({D, H});
  auto b1 = zeros<float>({H});
  auto W2 = random({H, D});
  auto b2 = zeros<float>({D});
  synchronize();
  return median_ms(reps, [&] {
    auto h1 = x.linear_sigmoid(W1, b1);
    auto out = h1.linear_sigmoid(W2, b2);
    eval(out);
    synchronize();
  });
}

// The reference's training benchmark (bench/composite/bench_train.cpp:20-58):
// a D -> H -> D MLP with sigmoid activations, MSE loss gradient, manual
// backward through sigmoid_backward, transposed products and sum(0), and an
// SGD update of all four parameters evaluated as one graph.
struct train_step {
  array<float> W1, b1, W2, b2, x, Y;
  float lr = 0.01f;
  size_t B, D, H;

  train_step(size_t batch, size_t d, size_t h, uint64_t seed) : B(batch), D(d), H(h) {
    rng g(seed);
    W1 = filled({D, H}, g, 0, true) * (1.0f / std::sqrt(float(D)));
    b1 = filled({H}, g, 0.1f);
    W2 = filled({H, D}, g, 0, true) * (1.0f / std::sqrt(float(H)));
    b2 = filled({D}, g, 0.1f);
    x = filled({B, D}, g, 0, true);
    Y = filled({B, D}, g, 0, true);
    eval(W1, W2);
  }

  // One step; leaves the updated parameters unevaluated in W1 .. b2.
  void step() {
    auto two = array<float>(2.0f);
    auto inv_n = array<float>(1.0f / static_cast<float>(B * D));
    auto neg_lr = array<float>(-lr);
    auto n1 = x.linear(W1, b1);
    auto o1 = n1.sigmoid();
    auto n2 = o1.linear(W2, b2);
    auto o2 = n2.sigmoid();
    auto dout = (o2 - Y) * two * inv_n;
    dout = n2.sigmoid_backward(dout);
    auto dW2 = o1.transpose().dot(dout);
    auto db2 = dout.sum(0);
    auto dout1 = dout.dot(W2.transpose());
    dout1 = n1.sigmoid_backward(dout1);
    auto dW1 = x.transpose().dot(dout1);
    auto db1 = dout1.sum(0);
    W1 = W1 + dW1 * neg_lr;
    b1 = b1 + db1 * neg_lr;
    W2 = W2 + dW2 * neg_lr;
    b2 = b2 + db2 * neg_lr;
  }

  // Six products of 2*B*D*H flops each (two forward, four backward).
  double gemm_flops() const { return 12.0 * double(B) * double(D) * double(H); }
};

void write_raw(const std::string &path, const array<float> &a) {
  std::ofstream f(path, std::ios::binary);
  const float *p = a.buffer_data();
  f.write(reinterpret_cast<const char *>(p), std::streamsize(a.element_count() * sizeof(float)));
  f.close();
  if (!f) throw std::runtime_error("cannot write " + path);
}

}  // namespace

// The reference's GPU micro-benchmarks, same operations and shapes, each
// iteration computing the result and waiting for it: element-wise add / mul /
// div / pow on ones (bench_elementwise.cpp:29-41, 249-258), the (N, M) + (M)
// bias broadcast (bench_broadcast.cpp:26-41), softmax and layer_norm of
// random rows (bench_nn_ops.cpp:24-35, 80-93), batched products
// (bench_nn_ops.cpp:252-270), full sum / min / max (bench_reduction.cpp:
// 28-34, 210-220; the scalar result is the wait), sum(0) and argmax of
// [m, 256] (bench_reduction.cpp:115-124, 290-300).
void micro() {
  auto report = [](const std::string &name, double ms) {
    std::printf("{\"workload\": \"micro\", \"name\": \"%s\", \"us\": %.2f}\n", name.c_str(),
                ms * 1e3);
    std::fflush(stdout);
  };
  const int reps = 50;
  for (auto [r, c] : {std::pair<size_t, size_t>{1024, 1024}, {4096, 512}, {4096, 4096}}) {
    auto a = ones<float>({r, c});
    auto b = ones<float>({c});
    array<float> y;
    report("broadcast (" + std::to_string(r) + "x" + std::to_string(c) + ")+(" +
               std::to_string(c) + ")",
           median_ms(reps, [&] {
             y = a + b;
             eval(y);
             synchronize();
           }));
  }
  for (size_t n : {size_t(1000000), size_t(10000000)}) {
    auto a = ones<float>({n});
    auto b = ones<float>({n});
    array<float> y;
    const std::string sz = " (" + std::to_string(n) + ")";
    report("add" + sz, median_ms(reps, [&] { y = a + b; eval(y); synchronize(); }));
    report("mul" + sz, median_ms(reps, [&] { y = a * b; eval(y); synchronize(); }));
    report("div" + sz, median_ms(reps, [&] { y = a / b; eval(y); synchronize(); }));
    report("pow" + sz, median_ms(reps, [&] { y = a.pow(b); eval(y); synchronize(); }));
  }
  for (auto [r, c] : {std::pair<size_t, size_t>{256, 512}, {1024, 1024}, {4096, 2048}, {256, 8192}}) {
    auto x = random({r, c});
    array<float> y;
    report("softmax (" + std::to_string(r) + "x" + std::to_string(c) + ")",
           median_ms(reps, [&] {
             y = x.softmax();
             eval(y);
             synchronize();
           }));
  }
  for (auto [r, c] : {std::pair<size_t, size_t>{256, 512}, {1024, 1024}, {4096, 2048}}) {
    auto x = random({r, c});
    auto gamma = ones<float>({c});
    auto beta = zeros<float>({c});
    array<float> y;
    report("layer_norm (" + std::to_string(r) + "x" + std::to_string(c) + ")",
           median_ms(reps, [&] {
             y = x.layer_norm(gamma, beta);
             eval(y);
             synchronize();
           }));
  }
  struct bm {
    size_t h, m, n, k;
  };
  for (auto [h, m, n, k] : {bm{8, 128, 128, 64}, bm{8, 512, 512, 64}, bm{16, 256, 256, 128}}) {
    auto a = random({h, m, k});
    auto b = random({h, k, n});
    array<float> y;
    report("bmm attention (" + std::to_string(h) + "h, seq=" + std::to_string(m) +
               ", d=" + std::to_string(k) + ")",
           median_ms(reps, [&] {
             y = a.batched_dot(b);
             eval(y);
             synchronize();
           }));
  }
  volatile float sink = 0.0f;
  for (size_t n : {size_t(1000000), size_t(10000000)}) {
    auto a = random({n});
    const std::string sz = " (" + std::to_string(n) + ")";
    report("sum" + sz, median_ms(reps, [&] { sink = a.sum(); }));
    report("min" + sz, median_ms(reps, [&] { sink = a.min(); }));
    report("max" + sz, median_ms(reps, [&] { sink = a.max(); }));
  }
  for (size_t m : {size_t(1024), size_t(4096)}) {
    auto a = random({m, size_t(256)});
    array<float> s;
    array<int> idx;
    const std::string sz = " (" + std::to_string(m) + "x256)";
    report("sum axis=0" + sz, median_ms(reps, [&] {
             s = a.sum(0);
             eval(s);
             synchronize();
           }));
    report("argmax" + sz, median_ms(reps, [&] {
             idx = a.argmax();
             eval(idx);
             synchronize();
           }));
  }
  (void)sink;
}

int main(int argc, char **argv) {
  const std::string mode = argc > 1 ? argv[1] : "encoder";
  try {
    if (mode == "micro") {
      micro();
      return 0;
    }
    if (mode == "chain") {
      const size_t n = argc > 2 ? std::strtoull(argv[2], nullptr, 10) : (size_t(64) << 20);
      const int reps = argc > 3 ? std::atoi(argv[3]) : 20;
      if (reps < 1 || n == 0) throw std::runtime_error("n and reps must be >= 1");
      rng g(7);
      auto x = filled({n}, g, 1.0f, true);
      auto run = [&] {
        auto y = x;
        for (int i = 0; i < 10; i++) y = y * (1.0f + 0.001f * float(i)) + (0.01f * float(i));
        eval(y);
      };
      const double ms = median_ms(reps, run);
      std::printf("{\"workload\": \"affine_chain20\", \"n\": %zu, \"ms\": %.4f, \"gbs\": %.1f}\n", n,
                  ms, 8.0 * double(n) / (ms * 1e-3) / 1e9);
      return 0;
    }
    if (mode == "transfer") {
      const size_t n = argc > 2 ? std::strtoull(argv[2], nullptr, 10) : (size_t(64) << 20);
      const int reps = argc > 3 ? std::atoi(argv[3]) : 10;
      if (reps < 1 || n == 0) throw std::runtime_error("n and reps must be >= 1");
      rng g(11);
      auto x = filled({n}, g, 1.0f, true);
      auto y = x * 2.0f;
      eval(y);
      const double copy_ms = median_ms(reps, [&] {  // the kernel alone
        auto t = x + 1.0f;
        eval(t);
      });
      float sink = 0.0f;
      // Upload: a host write makes the device copy stale, the next kernel
      // reading x uploads the whole mirror.
      const double up_ms = median_ms(reps, [&] {
        x.buffer_data()[0] += 1.0f;
        auto t = x + 1.0f;
        eval(t);
      });
      // Download: a fresh device result read on the host.
      const double down_ms = median_ms(reps, [&] {
        auto z = x * 2.0f;
        eval(z);
        sink += std::as_const(z).buffer_data()[n - 1];
      });
      const double gb = 4.0 * double(n) / 1e9;
      std::printf("{\"workload\": \"transfer\", \"n\": %zu, \"h2d_gbs\": %.1f, "
                  "\"d2h_gbs\": %.1f, \"kernel_ms\": %.4f, \"h2d_ms\": %.4f, "
                  "\"d2h_ms\": %.4f, \"check\": %d}\n",
                  n, gb / ((up_ms - copy_ms) * 1e-3), gb / ((down_ms - copy_ms) * 1e-3), copy_ms,
                  up_ms, down_ms, int(std::isfinite(sink)));
      return 0;
    }
    if (mode == "encoder" || mode == "encoder-dump") {
      // argv: mode [B S D H F [reps|DIR]] or, for "encoder", mode [reps].
      size_t dims[5] = {4, 512, 768, 12, 3072};
      const bool has_dims = argc >= 7;
      if (has_dims)
        for (int i = 0; i < 5; i++) dims[i] = std::strtoull(argv[2 + i], nullptr, 10);
      if (dims[3] == 0 || dims[2] % dims[3] != 0) {
        std::fprintf(stderr, "bench_graph: D must be a multiple of H\n");
        return 2;
      }
      encoder e(dims[0], dims[1], dims[2], dims[3], dims[4], 2026);
      if (mode == "encoder-dump") {
        const std::string dir = has_dims && argc > 7 ? argv[7] : ".";
        auto out = e.build();
        eval(out);
        // The same block with its intermediates held and evaluated in one
        // eval, so each stage can be checked against float64 computed from
        // this run's own fp32 inputs to that stage.
        auto st = e.stages();
        eval(st.out, st.h, st.qkv, st.merged, st.r1, st.h2, st.ff);
        write_raw(dir + "/h.bin", st.h);
        write_raw(dir + "/qkv.bin", st.qkv);
        write_raw(dir + "/merged.bin", st.merged);
        write_raw(dir + "/r1.bin", st.r1);
        write_raw(dir + "/h2.bin", st.h2);
        write_raw(dir + "/ff.bin", st.ff);
        write_raw(dir + "/out_staged.bin", st.out);
        write_raw(dir + "/x.bin", e.x);
        write_raw(dir + "/Wqkv.bin", e.Wqkv);
        write_raw(dir + "/bqkv.bin", e.bqkv);
        write_raw(dir + "/Wo.bin", e.Wo);
        write_raw(dir + "/bo.bin", e.bo);
        write_raw(dir + "/W1.bin", e.W1);
        write_raw(dir + "/c1.bin", e.c1);
        write_raw(dir + "/W2.bin", e.W2);
        write_raw(dir + "/c2.bin", e.c2);
        write_raw(dir + "/out.bin", out);
        std::printf("{\"dumped\": \"%s\"}\n", dir.c_str());
        return 0;
      }
      const int reps = has_dims ? (argc > 7 ? std::atoi(argv[7]) : 10)
                                : (argc > 2 ? std::atoi(argv[2]) : 10);
      if (reps < 1) {
        std::fprintf(stderr, "bench_graph: reps must be >= 1\n");
        return 2;
      }
      const double ms = median_ms(reps, [&] {
        auto out = e.build();
        eval(out);
      });
      std::printf(
          "{\"workload\": \"encoder_block\", \"B\": %zu, \"S\": %zu, \"D\": %zu, \"H\": %zu, "
          "\"F\": %zu, \"ms\": %.4f, \"gemm_tflops\": %.2f}\n",
          e.B, e.S, e.D, e.H, e.F, ms, e.gemm_flops() / (ms * 1e-3) / 1e12);
      return 0;
    }
    if (mode == "transformer") {
      // argv: [seq d_model d_ff [reps]]; default: the reference's four configs
      // (bench/composite/bench_transformer.cpp:77-82).
      std::vector<std::array<size_t, 3>> cfgs = {
          {256, 512, 2048}, {256, 768, 3072}, {256, 1024, 4096}, {512, 1024, 4096}};
      if (argc >= 5)
        cfgs = {{std::strtoull(argv[2], nullptr, 10), std::strtoull(argv[3], nullptr, 10),
                 std::strtoull(argv[4], nullptr, 10)}};
      const int reps = argc > 5 ? std::atoi(argv[5]) : 20;
      if (reps < 1) throw std::runtime_error("reps must be >= 1");
      for (auto [seq, d, f] : cfgs) {
        const double ms = transformer_ms(seq, d, f, reps);
        const double flops = 2.0 * seq * d * d * 4 + 2.0 * seq * seq * d * 2 + 2.0 * seq * d * f * 2;
        std::printf("{\"workload\": \"transformer_block\", \"seq\": %zu, \"d_model\": %zu, "
                    "\"d_ff\": %zu, \"ms\": %.4f, \"gemm_tflops\": %.2f}\n",
                    seq, d, f, ms, flops / (ms * 1e-3) / 1e12);
      }
      return 0;
    }
    if (mode == "mlp") {
      // argv: [batch [reps]]; default: the reference's batches 128, 256, 1024.
      std::vector<size_t> batches = {128, 256, 1024};
      if (argc >= 3) batches = {std::strtoull(argv[2], nullptr, 10)};
      const int reps = argc > 3 ? std::atoi(argv[3]) : 50;
      if (reps < 1) throw std::runtime_error("reps must be >= 1");
      for (size_t b : batches) {
        const double ms = mlp_ms(b, reps);
        const double flops = 2.0 * b * 768 * 2048 * 2;
        std::printf("{\"workload\": \"mlp_linear_sigmoid\", \"batch\": %zu, \"ms\": %.4f, "
                    "\"gemm_tflops\": %.2f}\n",
                    b, ms, flops / (ms * 1e-3) / 1e12);
      }
      return 0;
    }
    if (mode == "train") {
      // argv: [batch [reps]]; default: the reference's batches 64 and 128
      // (bench/composite/bench_train.cpp:60-64).
      std::vector<size_t> batches = {64, 128};
      if (argc >= 3) batches = {std::strtoull(argv[2], nullptr, 10)};
      const int reps = argc > 3 ? std::atoi(argv[3]) : 20;
      if (reps < 1 || batches[0] == 0) throw std::runtime_error("batch and reps must be >= 1");
      for (size_t b : batches) {
        train_step t(b, 768, 2048, 2027);
        synchronize();
        const double ms = median_ms(reps, [&] {
          t.step();
          eval(t.W1, t.b1, t.W2, t.b2);
          synchronize();
        });
        std::printf("{\"workload\": \"train_step\", \"batch\": %zu, \"D\": 768, \"H\": 2048, "
                    "\"ms\": %.4f, \"gemm_tflops\": %.2f}\n",
                    b, ms, t.gemm_flops() / (ms * 1e-3) / 1e12);
      }
      return 0;
    }
    if (mode == "mnist") {
      const size_t n_train = argc > 2 ? std::strtoull(argv[2], nullptr, 10) : 60000;
      const size_t n_test = argc > 3 ? std::strtoull(argv[3], nullptr, 10) : 10000;
      if (n_train < 100 || n_test < 1) throw std::runtime_error("need >= 100 training images");
      const auto r = mnist_bench(n_train, n_test);
      std::printf("{\"workload\": \"mnist\", \"train_images\": %zu, \"test_images\": %zu, "
                  "\"classifier_train_epoch_ms\": %.3f, \"classifier_inference_ms\": %.4f, "
                  "\"autoencoder_train_epoch_ms\": %.3f, \"autoencoder_inference_ms\": %.4f, "
                  "\"classifier_mse_first_batch\": [%.6f, %.6f]}\n",
                  n_train, n_test, r.classifier_train_ms, r.classifier_infer_ms,
                  r.autoencoder_train_ms, r.autoencoder_infer_ms, r.classifier_mse_first,
                  r.classifier_mse_last);
      return 0;
    }
    if (mode == "train-dump") {
      if (argc < 6) throw std::runtime_error("train-dump needs B D H DIR");
      const size_t B = std::strtoull(argv[2], nullptr, 10), D = std::strtoull(argv[3], nullptr, 10),
                   H = std::strtoull(argv[4], nullptr, 10);
      if (B == 0 || D == 0 || H == 0) throw std::runtime_error("B, D and H must be >= 1");
      const std::string dir = argv[5];
      train_step t(B, D, H, 2027);
      write_raw(dir + "/x.bin", t.x);
      write_raw(dir + "/Y.bin", t.Y);
      write_raw(dir + "/W1.bin", t.W1);
      write_raw(dir + "/b1.bin", t.b1);
      write_raw(dir + "/W2.bin", t.W2);
      write_raw(dir + "/b2.bin", t.b2);
      t.step();
      eval(t.W1, t.b1, t.W2, t.b2);
      write_raw(dir + "/W1_new.bin", t.W1);
      write_raw(dir + "/b1_new.bin", t.b1);
      write_raw(dir + "/W2_new.bin", t.W2);
      write_raw(dir + "/b2_new.bin", t.b2);
      std::printf("{\"dumped\": \"%s\"}\n", dir.c_str());
      return 0;
    }
    if (mode == "dot-dump") {
      if (argc < 6) throw std::runtime_error("dot-dump needs M N K DIR");
      const size_t M = std::strtoull(argv[2], nullptr, 10), N = std::strtoull(argv[3], nullptr, 10),
                   K = std::strtoull(argv[4], nullptr, 10);
      if (M == 0 || N == 0 || K == 0) throw std::runtime_error("M, N and K must be >= 1");
      const std::string dir = argv[5];
      rng g(2028);
      auto A = filled({M, K}, g, 1.0f, true);
      auto B = filled({K, N}, g, 1.0f, true);
      auto C = A.dot(B);
      eval(C);
      write_raw(dir + "/A.bin", A);
      write_raw(dir + "/B.bin", B);
      write_raw(dir + "/C.bin", C);
      std::printf("{\"dumped\": \"%s\"}\n", dir.c_str());
      return 0;
    }
    if (mode == "chain-dump") {
      if (argc < 4) throw std::runtime_error("chain-dump needs n DIR");
      const size_t n = std::strtoull(argv[2], nullptr, 10);
      if (n == 0) throw std::runtime_error("n must be >= 1");
      const std::string dir = argv[3];
      rng g(7);
      auto x = filled({n}, g, 1.0f, true);
      auto y = x;
      for (int i = 0; i < 10; i++) y = y * (1.0f + 0.001f * float(i)) + (0.01f * float(i));
      eval(y);
      write_raw(dir + "/x.bin", x);
      write_raw(dir + "/y.bin", y);
      std::printf("{\"dumped\": \"%s\"}\n", dir.c_str());
      return 0;
    }
    std::fprintf(stderr,
                 "usage: bench_graph chain|transfer|mnist|encoder|encoder-dump|transformer|mlp|"
                 "train|train-dump|dot-dump|chain-dump ...\n");
    return 2;
  } catch (std::exception &ex) {
    std::fprintf(stderr, "bench_graph: %s\n", ex.what());
    return 1;
  }
}
