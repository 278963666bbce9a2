// C++ front-end tests: the behaviour the reference's doctest suite pins
// (test/test_array.cpp, test/test_examples.cpp, test/test_2lnn.cpp) checked
// against this build's sil::array on the MI355X backend, plus checks of
// the eval() lowering (fusion, reference rounding of scalar chains) and the
// storage/host-mirror protocol.  HOST_CASEs touch no GPU and run in the CPU
// test suite; TEST_CASEs need the GPU.
#include <silarray.h>

#include <cmath>
#include <cstring>
#include <numeric>
#include <tuple>
#include <ranges>
#include <utility>
#include <vector>

#include "harness.h"

using namespace sil;

static auto iota_n(size_t n, int start = 1) {
  return std::views::iota(start) | std::views::take(n);
}

//------------------------------------------------------------------------------
// Shapes, views, host-side logic (no GPU)
//------------------------------------------------------------------------------

HOST_CASE("scalar shape") {
  auto s = array<int>(100);
  CHECK(s.element_count() == 1);
  CHECK(s.dimension() == 0);
  CHECK(s.shape() == shape_type{});
  CHECK(s.at() == 100);
  CHECK_THROWS_WITH(s.length(), "array: cannot call with a scalar value.");
}

HOST_CASE("vector shape and construction") {
  auto v = empty<int>({3});
  CHECK(v.element_count() == 3 && v.length() == 3 && v.dimension() == 1);
  auto w = array<int>{1, 2, 3, 4};
  CHECK(w.element_count() == 4);
  std::vector<int> src{1, 2, 3, 4};
  auto v1 = array<int>({src.size() - 1}, src);
  CHECK(array_equal(v1, {1, 2, 3}));
  auto v3 = array<int>(src);
  CHECK(array_equal(v3, {1, 2, 3, 4}));
  auto r = array<int>({10}, iota_n(10));
  CHECK(array_equal(r, {1, 2, 3, 4, 5, 6, 7, 8, 9, 10}));
}

HOST_CASE("matrix and tensor initializers") {
  auto m2 = array<int>{{1, 2, 3, 4}, {5, 6, 7, 8}, {9, 10, 11, 12}};
  CHECK(m2.shape() == (shape_type{3, 4}));
  CHECK(m2.strides() == (strides_type{4, 1}));
  auto m3 = array<int>{{{1, 2, 3}, {4, 5, 6}}, {{7, 8, 9}, {10, 11, 12}}};
  CHECK(m3.shape() == (shape_type{2, 2, 3}));
  CHECK(m3.strides() == (strides_type{6, 3, 1}));
  CHECK_THROWS_WITH((array<int>{{{1, 2, 3}, {4, 5}}, {{7, 8, 9}, {10, 11, 12}}}),
                    "array: invalid initializer list.");
  auto m = array<int>({3, 4}, iota_n(12));
  size_t i = 0;
  for (size_t r = 0; r < 3; r++)
    for (size_t c = 0; c < 4; c++) CHECK((m[r, c]) == m.at(i++));
}

HOST_CASE("bounds checks") {
  auto v = array<int>({10}, iota_n(10, 0));
  CHECK(v.at(9) == 9);
  CHECK_THROWS_WITH(v.at(10), "array: index is out of bounds.");
  auto t = array<int>{{{1, 2, 3}, {4, 5, 6}}};
  CHECK_THROWS_WITH(t[3], "array: row is out of bounds.");
  // layer_norm reads one gamma and one beta per column: other lengths are
  // refused when the node is built, before any kernel could read past them
  auto x = array<float>({2, 4}, std::vector<float>{1, 2, 3, 4, 5, 6, 7, 8});
  auto g4 = array<float>({4}, std::vector<float>{1, 1, 1, 1});
  auto g3 = array<float>({3}, std::vector<float>{1, 1, 1});
  CHECK_THROWS_WITH(x.layer_norm(g3, g4), "array: layer_norm needs one gamma and one beta per column.");
  CHECK_THROWS_WITH(x.layer_norm(g4, g3), "array: layer_norm needs one gamma and one beta per column.");
  CHECK_THROWS_WITH(array<float>({3}, std::vector<float>{1, 2, 3}).layer_norm(g3, g3),
                    "array: layer_norm requires 2D array.");
}

HOST_CASE("transpose views") {
  auto v = array<int>{1, 2, 3, 4};
  auto vT = v.transpose();
  CHECK(vT.shape() == (shape_type{1, 4}));
  CHECK(array_equal(vT, {{1, 2, 3, 4}}));
  CHECK(array_equal(vT.transpose(), {1, 2, 3, 4}));
  auto m = array<int>{{1, 2, 3, 4}, {5, 6, 7, 8}, {9, 10, 11, 12}};
  auto mT = m.transpose();
  CHECK(mT.shape() == (shape_type{4, 3}));
  CHECK(array_equal(mT, {{1, 5, 9}, {2, 6, 10}, {3, 7, 11}, {4, 8, 12}}));
  CHECK(array_equal(mT.transpose(), m));
  auto t = array<int>{{{1, 2, 3, 4}, {5, 6, 7, 8}}, {{9, 10, 11, 12}, {13, 14, 15, 16}}};
  auto tT = t.transpose();
  CHECK(tT.shape() == (shape_type{4, 2, 2}));
  CHECK(array_equal(tT.transpose(), t));
  // A row of a transposed view is a {1, n} view that is not contiguous: its
  // transpose is the vector {n} (as for any row) holding that row's elements.
  auto row = mT.slice(2, 1);  // {{3, 7, 11}}, strides {1, 4}
  CHECK(array_equal(row, {{3, 7, 11}}));
  auto rowT = row.transpose();
  CHECK(rowT.shape() == (shape_type{3}));
  CHECK(array_equal(rowT, {3, 7, 11}));
}

HOST_CASE("broadcast view") {
  auto a = array<int>{{1, 2, 3}, {4, 5, 6}};
  auto b = a.broadcast({3, 2, 3});
  CHECK(array_equal(b, {{{1, 2, 3}, {4, 5, 6}}, {{1, 2, 3}, {4, 5, 6}}, {{1, 2, 3}, {4, 5, 6}}}));
  CHECK(b.element_count() == 18);
  CHECK(b.buffer_element_count() == 6);
  CHECK((b[2, 1, 2]) == 6);
  CHECK(b.strides() == (strides_type{0, 3, 1}));
}

HOST_CASE("row views share storage") {
  auto t = array<int>{{{1, 2, 3}, {4, 5, 6}}, {{7, 8, 9}, {10, 11, 12}}, {{13, 14, 15}, {16, 17, 18}}};
  auto m = t[1];
  auto v = m[1];
  auto s = v[1];
  CHECK(array_equal(m, {{7, 8, 9}, {10, 11, 12}}));
  CHECK(array_equal(s, array<int>(11)));
  s.at() += 100;
  CHECK(array_equal(t, {{{1, 2, 3}, {4, 5, 6}}, {{7, 8, 9}, {10, 111, 12}}, {{13, 14, 15}, {16, 17, 18}}}));
  m.zeros();
  CHECK(array_equal(v, {0, 0, 0}));
  CHECK(array_equal(t, {{{1, 2, 3}, {4, 5, 6}}, {{0, 0, 0}, {0, 0, 0}}, {{13, 14, 15}, {16, 17, 18}}}));
}

HOST_CASE("int aggregates") {
  auto v = array<int>{1, 2, 3, 4, 5, 6};
  auto t = array<int>{{{1, 2, 3}, {4, 5, 6}}, {{7, 8, 9}, {10, 11, 12}}, {{13, 14, 15}, {16, 17, 18}}};
  CHECK(v.min() == 1 && v.max() == 6 && t.min() == 1 && t.max() == 18);
  CHECK(v.sum() == 21 && t.sum() == 171);
  CHECK(array_equal(t.sum(0), {{21, 24, 27}, {30, 33, 36}}));
  CHECK(array_equal(t.sum(1), {{5, 7, 9}, {17, 19, 21}, {29, 31, 33}}));
  CHECK(array_equal(t.sum(2), {{6, 15}, {24, 33}, {42, 51}}));
  CHECK(v.mean() == 3.5f && t.mean() == 9.5f);
  auto row = array<int>{{10, 20, 30}, {1, 2, 3}}[1];
  CHECK(row.min() == 1 && row.max() == 3 && row.count() == 3 && !row.all(1));
}

HOST_CASE("iterators") {
  auto t = array<int>{{{1, 2, 3}, {4, 5, 6}}, {{7, 8, 9}, {10, 11, 12}}, {{13, 14, 15}, {16, 17, 18}}};
  for (auto row : t)
    for (auto &x : row.elements()) x += 100;
  const auto ct = t;
  int cur = 101;
  for (auto row : ct.rows())
    for (const auto &x : row.elements()) CHECK(x == cur++);
  cur = 101;
  for (auto row : ct.rows())
    for (auto [a, b, c] : row.rows<3>()) {
      CHECK(a == cur++);
      CHECK(b == cur++);
      CHECK(c == cur++);
    }
}

HOST_CASE("int argmax, one_hot, where") {
  auto m = array<int>{{3, 1, 2}, {6, 8, 7}};
  CHECK(array_equal(m.argmax(), {0, 1}));
  auto v = array<float>{0, 1, 5, 9};
  auto oh = v.one_hot(10);
  CHECK(oh.shape() == (shape_type{4, 10}));
  CHECK((oh[2, 5]) == 1.0f && (oh[2, 4]) == 0.0f && (oh[3, 9]) == 1.0f);
  auto w = where(array<int>{1, 0, 2} > array<int>(0), 5, 7);
  CHECK(array_equal(w, {5, 7, 5}));
}

HOST_CASE("int arithmetic in CPU mode") {
  use_cpu();
  auto a = array<int>({3, 4}, iota_n(12));
  auto b = array<int>({3, 4}, iota_n(12));
  CHECK(array_equal(a + b, {{2, 4, 6, 8}, {10, 12, 14, 16}, {18, 20, 22, 24}}));
  CHECK(array_equal(a * b, {{1, 4, 9, 16}, {25, 36, 49, 64}, {81, 100, 121, 144}}));
  CHECK(array_equal(a / b, {{1, 1, 1, 1}, {1, 1, 1, 1}, {1, 1, 1, 1}}));
  CHECK(array_equal(array<int>{1, 2, 3}.pow(array<int>{2, 2, 2}), {1, 4, 9}));
  auto c = array<int>({3, 1}, std::vector{1, 2, 3}) + array<int>({1, 3}, std::vector{10, 20, 30});
  CHECK(array_equal(c, {{11, 21, 31}, {12, 22, 32}, {13, 23, 33}}));
  // float evaluation is GPU-only in this build
  CHECK_THROWS_WITH((array<float>{1.0f} + array<float>{2.0f}).at(0),
                    "array: float evaluation needs the GPU backend (sil::use_gpu()); the CPU "
                    "backend is not part of this build.");
  use_gpu();
}

//------------------------------------------------------------------------------
// GPU: elementwise, broadcast, scalars
//------------------------------------------------------------------------------

TEST_CASE("float vector arithmetic goldens") {
  auto a = array<float>{7.82637e-06, 0.131538, 0.755605, 0.45865, 0.532767, 0.218959, 0.0470446,
                        0.678865, 0.679296, 0.934693, 0.383502, 0.519416, 0.830965, 0.0345721,
                        0.0534616, 0.5297};
  auto b = array<float>{0.671149, 0.00769819, 0.383416, 0.0668422, 0.417486, 0.686773, 0.588977,
                        0.930436, 0.846167, 0.526929, 0.0919649, 0.653919, 0.415999, 0.701191,
                        0.910321, 0.762198};
  CHECK(allclose(a + b, {0.671157, 0.139236, 1.13902, 0.525492, 0.950253, 0.905732, 0.636021,
                         1.6093, 1.52546, 1.46162, 0.475467, 1.17334, 1.24696, 0.735763,
                         0.963782, 1.2919}));
  CHECK(allclose(a - b, {-0.671141, 0.12384, 0.372189, 0.391808, 0.115281, -0.467814, -0.541932,
                         -0.251571, -0.166871, 0.407764, 0.291537, -0.134503, 0.414966, -0.666619,
                         -0.856859, -0.232498}));
  CHECK(allclose(a * b, {5.25266e-06, 0.0010126, 0.289711, 0.0306572, 0.222423, 0.150375,
                         0.0277082, 0.63164, 0.574798, 0.492517, 0.0352687, 0.339656, 0.345681,
                         0.0242416, 0.0486672, 0.403736}));
  CHECK(allclose(a / b, {1.16612e-05, 17.0869, 1.97072, 6.86168, 1.27613, 0.318823, 0.0798751,
                         0.72962, 0.802792, 1.77385, 4.17009, 0.794312, 1.99752, 0.0493048,
                         0.0587283, 0.694964}));
  CHECK_THROWS_WITH(random({4}) + random({8}), "array: invalid operation.");
}

TEST_CASE("pow int and float") {
  CHECK(array_equal(array<int>{1, 2, 3}.pow(array<int>{2, 2, 2}), {1, 4, 9}));
  CHECK(array_equal(array<int>{2, 2, 2}.pow(array<int>{1, 2, 3}), {2, 4, 8}));
  CHECK(allclose(array<float>{1, 2, 3}.pow(array<float>{2, 2, 2}), {1, 4, 9}));
  CHECK(allclose(array<float>{2, 2, 2}.pow(array<float>{1, 2, 3}), {2, 4, 8}));
}

TEST_CASE("int matrix arithmetic on the GPU") {
  auto a = array<int>({3, 4}, iota_n(12));
  auto b = array<int>({3, 4}, iota_n(12));
  CHECK(array_equal(a + b, {{2, 4, 6, 8}, {10, 12, 14, 16}, {18, 20, 22, 24}}));
  CHECK(array_equal(a - b, {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}}));
  CHECK(array_equal(a * b, {{1, 4, 9, 16}, {25, 36, 49, 64}, {81, 100, 121, 144}}));
  CHECK(array_equal(a / b, {{1, 1, 1, 1}, {1, 1, 1, 1}, {1, 1, 1, 1}}));
}

TEST_CASE("scalar arithmetic") {
  auto a = array<float>{{1, 2}, {3, 4}};
  CHECK(array_equal(a + 1, {{2, 3}, {4, 5}}));
  CHECK(array_equal(a - 1, {{0, 1}, {2, 3}}));
  CHECK(array_equal(a * 2, {{2, 4}, {6, 8}}));
  CHECK(array_equal(a / 2, {{0.5, 1}, {1.5, 2}}));
  CHECK(array_equal(1 + a, {{2, 3}, {4, 5}}));
  CHECK(array_equal(1 - a, {{0, -1}, {-2, -3}}));
  CHECK(array_equal(2 * a, {{2, 4}, {6, 8}}));
  CHECK(array_equal(2 / a, {{2, 1}, {2.0f / 3.0f, 0.5}}));
}

TEST_CASE("broadcast arithmetic") {
  auto a23 = array<int>{{1, 2, 3}, {4, 5, 6}};
  auto a223 = array<int>{{{1, 2, 3}, {4, 5, 6}}, {{7, 8, 9}, {10, 11, 12}}};
  auto b = array<int>(1);
  auto b3 = array<int>{1, 2, 3};
  auto b23 = array<int>{{1, 2, 3}, {4, 5, 6}};
  CHECK(array_equal(a23 + b, {{2, 3, 4}, {5, 6, 7}}));
  CHECK(array_equal(a223 + b3, {{{2, 4, 6}, {5, 7, 9}}, {{8, 10, 12}, {11, 13, 15}}}));
  CHECK(array_equal(a223 + b23, {{{2, 4, 6}, {8, 10, 12}}, {{8, 10, 12}, {14, 16, 18}}}));
  CHECK(array_equal(b3 + a23, {{2, 4, 6}, {5, 7, 9}}));
  CHECK(array_equal(b23 + a223, {{{2, 4, 6}, {8, 10, 12}}, {{8, 10, 12}, {14, 16, 18}}}));
  auto c = array<int>({3, 1}, std::vector{1, 2, 3}) + array<int>({1, 3}, std::vector{10, 20, 30});
  CHECK(array_equal(c, {{11, 21, 31}, {12, 22, 32}, {13, 23, 33}}));
  // float, including a middle-axis broadcast the i % len rule cannot express
  auto f = array<float>({2, 2, 3}, iota_n(12)) * array<float>({2, 1, 3}, iota_n(6));
  CHECK(array_equal(f, {{{1, 4, 9}, {4, 10, 18}}, {{28, 40, 54}, {40, 55, 72}}}));
}

TEST_CASE("sigmoid and relu") {
  auto s = array<float>{0.0f, 1.0f, -1.0f, 5.0f, -5.0f}.sigmoid();
  CHECK(is_close(s.at(0), 0.5f) && is_close(s.at(1), 0.7310f) && is_close(s.at(2), 0.2689f));
  CHECK(s.at(3) > 0.99f && s.at(4) < 0.01f);
  auto big = random({64, 128}).sigmoid();
  CHECK(big.all([](float x) { return x >= 0.0f && x <= 1.0f; }));
  auto r = array<float>{-2.0f, -1.0f, 0.0f, 1.0f, 2.0f}.relu();
  CHECK(array_equal(r, {0.0f, 0.0f, 0.0f, 1.0f, 2.0f}));
  auto br = (random({64, 128}) - array<float>(0.5f)).relu();
  CHECK(br.all([](float x) { return x >= 0.0f; }));
}

//------------------------------------------------------------------------------
// GPU: products
//------------------------------------------------------------------------------

TEST_CASE("dot goldens") {
  CHECK(array_equal(array<int>({4}, iota_n(4)).dot(array<int>({4}, iota_n(4))), array<int>(30)));
  CHECK(array_equal(array<int>({3, 4}, iota_n(12)).dot(array<int>({4, 2}, iota_n(8))),
                    {{50, 60}, {114, 140}, {178, 220}}));
  auto fa = array<float>({3, 4}, std::vector<float>{1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12});
  auto fb = array<float>({4, 2}, std::vector<float>{1, 2, 3, 4, 5, 6, 7, 8});
  auto fo = fa.dot(fb);
  CHECK(fo.shape() == (shape_type{3, 2}));
  CHECK(array_equal(fo, {{50, 60}, {114, 140}, {178, 220}}));
  CHECK(array_equal(array<float>({4}, iota_n(4)).dot(array<float>({4, 2}, iota_n(8))), {50, 60}));
  CHECK(array_equal(array<float>({2, 4}, iota_n(8)).dot(array<float>({4}, iota_n(4))), {30, 70}));
  auto vv = array<float>({4}, iota_n(4)).dot(array<float>({4}, iota_n(4)));
  CHECK(vv.shape() == shape_type{} && vv.at() == 30.0f);
  auto y = array<float>{1, 2, 3}.dot(array<float>{{1, 2}, {3, 4}, {5, 6}});
  CHECK(array_equal(y, {22, 28}));
}

TEST_CASE("dot with transposed views") {
  auto x = ones<float>({4, 3});
  auto dout = ones<float>({4, 2});
  auto W = ones<float>({3, 2}) * 0.5f;
  auto dx = dout.dot(W.transpose());
  CHECK(dx.shape() == (shape_type{4, 3}));
  CHECK(dx.all([](float v) { return std::abs(v - 1.0f) < 1e-6f; }));
  auto dW = x.transpose().dot(dout);
  CHECK(dW.shape() == (shape_type{3, 2}));
  CHECK(dW.all([](float v) { return std::abs(v - 4.0f) < 1e-6f; }));
}

TEST_CASE("linear and linear_sigmoid") {
  auto x = array<float>({2, 3}, std::vector<float>{1, 2, 3, 4, 5, 6});
  auto W = array<float>({3, 2}, std::vector<float>{1, 2, 3, 4, 5, 6});
  auto b = array<float>({2}, std::vector<float>{10, 20});
  auto out = x.linear(W, b);
  CHECK(array_equal(out, {{32, 48}, {59, 84}}));
  auto out2 = out.sigmoid().linear(array<float>({2, 1}, std::vector<float>{1, 1}),
                                   array<float>({1}, std::vector<float>{0}));
  CHECK(out2.shape() == (shape_type{2, 1}));
  CHECK(std::abs(*out2.element_cbegin() - 2.0f) < 0.02f);
  auto ls = x.linear_sigmoid(W, b);
  CHECK(ls.all([](float v) { return v > 0.999f; }));
}

TEST_CASE("batched_dot") {
  auto a = array<float>({2, 2, 3}, iota_n(12));
  auto b = array<float>({2, 3, 2}, iota_n(12));
  auto c = a.batched_dot(b);
  CHECK(c.shape() == (shape_type{2, 2, 2}));
  CHECK(array_equal(c, {{{22, 28}, {49, 64}}, {{220, 244}, {301, 334}}}));
}

//------------------------------------------------------------------------------
// GPU: reductions and row ops
//------------------------------------------------------------------------------

TEST_CASE("float aggregates") {
  CHECK(is_close(array<float>{1.1f, 2.2f}.sum(), 3.3f));
  CHECK(is_close(ones<float>({10000}).sum(), 10000.0f, 1.0f));
  auto big2d = ones<float>({256, 128});
  CHECK(is_close(big2d.sum(), 32768.0f, 1.0f));
  auto s0 = big2d.sum(0);
  CHECK(s0.shape() == shape_type{128} && is_close(s0.at(0), 256.0f, 1.0f));
  auto t = array<float>({3, 2, 3}, iota_n(18));
  CHECK(array_equal(t.sum(0), {{21, 24, 27}, {30, 33, 36}}));
  CHECK(array_equal(t.sum(1), {{5, 7, 9}, {17, 19, 21}, {29, 31, 33}}));
  CHECK(array_equal(t.sum(2), {{6, 15}, {24, 33}, {42, 51}}));
  CHECK(array_equal(t.mean(0), {{7, 8, 9}, {10, 11, 12}}));
  CHECK(array_equal(t.mean(2), {{2, 5}, {8, 11}, {14, 17}}));
  CHECK(t.min() == 1.0f && t.max() == 18.0f && t.mean() == 9.5f);
  auto fm = array<float>{{3, 1, 2}, {6, 8, 7}};
  CHECK(array_equal(fm.argmax(), {0, 1}));
  CHECK((array<float>{1, 2, 3, 4}.mean_square_error(array<float>{0, 2, 3, 6}) == 1.25f));
}

TEST_CASE("layer_norm") {
  auto x = array<float>{{1.0f, 2.0f, 3.0f}, {4.0f, 5.0f, 6.0f}};
  auto out = x.layer_norm(array<float>{1, 1, 1}, array<float>{0, 0, 0});
  CHECK(out.shape() == (shape_type{2, 3}));
  CHECK(is_close((out[0, 0]), -1.2247f, 1e-2f) && is_close((out[0, 1]), 0.0f, 1e-2f) &&
        is_close((out[0, 2]), 1.2247f, 1e-2f));
  auto out2 = x.layer_norm(array<float>{2, 2, 2}, array<float>{1, 1, 1});
  CHECK(is_close((out2[0, 1]), 1.0f, 1e-2f));
  auto big = random({64, 256}).layer_norm(ones<float>({256}), zeros<float>({256}));
  for (size_t i = 0; i < 64; i++) CHECK(is_close(big[i].mean(), 0.0f, 0.1f));
}

TEST_CASE("softmax") {
  auto vsm = array<int>{1, 2, 3, 4, 5, 6}.softmax();
  CHECK(is_close(vsm.sum(), 1.0f, 1e-6f));
  auto msm = array<int>{{7, 8, 9}, {10, 11, 12}}.softmax();
  CHECK(allclose(msm.sum(1), array<float>{1, 1}, 1e-6f));
  auto sm = array<float>{1.0f, 2.0f, 3.0f}.softmax();
  CHECK(is_close(sm.at(0), 0.0900f) && is_close(sm.at(1), 0.2447f) && is_close(sm.at(2), 0.6652f));
  auto big = random({64, 32}).softmax();
  for (size_t i = 0; i < 64; i++) CHECK(is_close(big[i].sum(), 1.0f, 1e-3f));
}

//------------------------------------------------------------------------------
// GPU: eval() lowering
//------------------------------------------------------------------------------

TEST_CASE("affine chain fuses and keeps reference rounding") {
  // 20 scalar affine nodes on one array: one fused launch whose result
  // equals node-by-node evaluation with the reference's folding
  // (mul -> fma(x, s, 0), add -> fma(x, 1, b), div -> fma(x, 1/r, 0)).
  const size_t n = 1 << 20;
  auto x = random({n});
  std::vector<float> host(x.buffer_data(), x.buffer_data() + n);
  auto y = x;
  for (int i = 0; i < 10; i++) y = y * (1.0f + 0.01f * i) + (0.001f * i);
  y = y / 3.0f - 0.5f;
  eval(y);
  std::vector<float> ref = host;
  for (auto &v : ref) {
    for (int i = 0; i < 10; i++) {
      v = std::fma(v, 1.0f + 0.01f * i, 0.0f * (1.0f + 0.01f * i));
      v = std::fma(v, 1.0f, 0.0f + 0.001f * i);
    }
    v = std::fma(v, 1.0f / 3.0f, 0.0f / 3.0f);
    v = std::fma(v, 1.0f, 0.0f - 0.5f);
  }
  bool same = true;
  const float *p = y.buffer_data();
  for (size_t i = 0; i < n; i++) same = same && (p[i] == ref[i]);
  CHECK(same);
}

TEST_CASE("fused graph with shared and broadcast operands") {
  auto a = random({33, 129});
  auto b = random({129});
  auto c = random({33, 1});
  auto t = (a * b + c).relu();       // intermediate used twice -> materialised
  auto u = t * t - t.sigmoid() / 2.0f;
  eval(u, t);
  const float *pa = a.buffer_data(), *pb = b.buffer_data(), *pc = c.buffer_data();
  bool ok = true;
  for (size_t i = 0; i < 33; i++)
    for (size_t j = 0; j < 129; j++) {
      float tv = std::max(pa[i * 129 + j] * pb[j] + pc[i], 0.0f);
      float s = 1.0f / (1.0f + std::exp(-tv));
      float uv = tv * tv - std::fma(s, 0.5f, 0.0f * 0.5f);
      ok = ok && std::abs((t[i, j]) - tv) <= 1e-6f && std::abs((u[i, j]) - uv) <= 2e-6f;
    }
  CHECK(ok);
}

TEST_CASE("arrays held outside the graph are materialised") {
  auto x = random({1000});
  auto y = x * 2.0f;      // held by `y`
  auto z = y + 1.0f;
  eval(z);
  CHECK(y.lazy_node_ptr()->evaluated);
  bool ok = true;
  for (size_t i = 0; i < 1000; i++) ok = ok && (y.at(i) == x.at(i) * 2.0f) && (z.at(i) == y.at(i) + 1.0f);
  CHECK(ok);
}

TEST_CASE("a product evaluated early, then added in a later eval") {
  // A row view of a lazy product (slice) evaluates the product and frees
  // its graph inputs; the add that consumes it afterwards must not try to
  // fold it into the product's epilogue (that read the freed inputs).
  auto x = array<float>({2, 3}, std::vector<float>{1, 2, 3, 4, 5, 6});
  auto W = array<float>({3, 3}, std::vector<float>{1, 0, 0, 0, 1, 0, 0, 0, 1});
  auto b = array<float>({3}, std::vector<float>{10, 20, 30});
  auto lin = x.linear(W, b);
  auto prod = x.dot(W);
  auto first = lin.slice(0, 1);   // evaluates lin
  auto firstp = prod.slice(1, 1); // evaluates prod
  auto r1 = x + lin;
  auto r2 = prod + x;
  auto r3 = lin.relu() + 1.0f;
  eval(r1, r2, r3);
  CHECK(array_equal(first, {{11, 22, 33}}));
  CHECK(array_equal(firstp, {{4, 5, 6}}));
  CHECK(array_equal(r1, {{12, 24, 36}, {18, 30, 42}}));
  CHECK(array_equal(r2, {{2, 4, 6}, {8, 10, 12}}));
  CHECK(array_equal(r3, {{12, 23, 34}, {15, 26, 37}}));
}

TEST_CASE("eval of a root that another root consumes") {
  // Both roots are products; the second consumes the first, so the first
  // must be computed before it even though both are requested together.
  auto x = array<float>({2, 3}, std::vector<float>{1, 2, 3, 4, 5, 6});
  auto W = array<float>({3, 2}, std::vector<float>{1, 2, 3, 4, 5, 6});
  auto W2 = array<float>({2, 1}, std::vector<float>{1, -1});
  auto a = x.dot(W);
  auto b = a.dot(W2);
  eval(a, b);
  CHECK(array_equal(a, {{22, 28}, {49, 64}}));
  CHECK(array_equal(b, {{-6}, {-15}}));
}

TEST_CASE("product with the transpose of a lazy matrix") {
  // scores = Q K^T as the reference's transformer writes it
  // (bench/composite/bench_transformer.cpp:60): K^T stays a lazy view.
  auto x = random({20, 12});
  auto Wq = random({12, 8}) - 0.5f, Wk = random({12, 8}) - 0.5f;
  auto bq = random({8}), bk = random({8});
  eval(x, Wq, Wk, bq, bk);
  auto Q = x.linear(Wq, bq);
  auto K = x.linear(Wk, bk);
  auto Kt = K.transpose();
  CHECK(Kt.shape() == (shape_type{8, 20}));
  auto s = Q.dot(Kt) * 0.5f;
  eval(s, Q, K);
  bool ok = true;
  for (size_t i = 0; i < 20; i++)
    for (size_t j = 0; j < 20; j++) {
      double acc = 0;
      for (size_t e = 0; e < 8; e++) acc += double(Q[i, e]) * double(K[j, e]);
      ok = ok && std::abs((s[i, j]) - 0.5 * acc) <= 1e-5 * (1 + std::abs(acc));
    }
  CHECK(ok);
}

TEST_CASE("scalar and residual nodes fused into products stay bit-exact") {
  // Each fused graph is compared with the same graph evaluated with the
  // intermediate held by an array (held nodes are never fused).
  auto x = random({70, 48}) - 0.5f;
  auto W = random({48, 33}) - 0.5f;
  auto b = random({33}) - 0.5f;
  auto r = random({70, 33}) - 0.5f;
  auto q = random({2, 3, 5, 8}) - 0.5f, k = random({2, 3, 8, 5}) - 0.5f;
  eval(x, W, b, r, q, k);
  auto same = [](const array<float> &a, const array<float> &c) {
    if (a.shape() != c.shape()) return false;
    const float *pa = a.buffer_data(), *pc = c.buffer_data();
    for (size_t i = 0; i < a.element_count(); i++)
      if (std::memcmp(&pa[i], &pc[i], sizeof(float)) != 0) return false;
    return true;
  };
  {  // dot * s, s - dot, dot / s
    auto f1 = x.dot(W) * 0.3f, f2 = 1.5f - x.dot(W), f3 = x.dot(W) / 7.0f;
    eval(f1, f2, f3);
    auto held = x.dot(W);
    eval(held);
    auto u1 = held * 0.3f, u2 = 1.5f - held, u3 = held / 7.0f;
    eval(u1, u2, u3);
    CHECK(same(f1, u1) && same(f2, u2) && same(f3, u3));
  }
  {  // batched_dot * s over a two-level batch
    auto f = q.batched_dot(k) * 0.125f;
    eval(f);
    auto held = q.batched_dot(k);
    eval(held);
    auto u = held * 0.125f;
    eval(u);
    CHECK(same(f, u));
  }
  {  // r + linear, linear + r, r + relu(linear), r + dot
    auto f1 = r + x.linear(W, b), f2 = x.linear(W, b) + r, f3 = r + x.linear(W, b).relu();
    auto f4 = r + x.dot(W);
    eval(f1, f2, f3, f4);
    auto h1 = x.linear(W, b), h3 = x.linear(W, b).relu(), h4 = x.dot(W);
    eval(h1, h3, h4);
    auto u1 = r + h1, u2 = h1 + r, u3 = r + h3, u4 = r + h4;
    eval(u1, u2, u3, u4);
    CHECK(same(f1, u1) && same(f2, u2) && same(f3, u3) && same(f4, u4));
  }
}

TEST_CASE("lazy views feed strided batched products") {
  // qkv [B*S, 3*H*dh] split into heads by view/permute/select, as an
  // attention block does; every product reads its operand in place.
  const size_t B = 2, S = 3, H = 2, dh = 4, D = H * dh;
  auto qkv = random({B * S, 3 * D});
  auto heads = (qkv * 1.0f).view({B, S, 3, H, dh}).permute({2, 0, 3, 1, 4});
  CHECK(heads.shape() == (shape_type{3, B, H, S, dh}));
  auto q = heads.select(0, 0), k = heads.select(0, 1), v = heads.select(0, 2);
  auto scores = q.batched_dot(k.permute({0, 1, 3, 2}));
  auto ctx = scores.batched_dot(v);
  auto merged = ctx.permute({0, 2, 1, 3}).view({B * S, D});
  eval(scores, merged);
  CHECK(scores.shape() == (shape_type{B, H, S, S}) && merged.shape() == (shape_type{B * S, D}));
  const float *p = std::as_const(qkv).buffer_data();
  const float *ps = std::as_const(scores).buffer_data();
  auto at = [&](size_t part, size_t b, size_t h, size_t s, size_t e) {
    return double(p[(b * S + s) * 3 * D + part * D + h * dh + e]);
  };
  bool ok = true;
  for (size_t b = 0; b < B; b++)
    for (size_t h = 0; h < H; h++)
      for (size_t i = 0; i < S; i++) {
        double sc[S];
        for (size_t j = 0; j < S; j++) {
          sc[j] = 0;
          for (size_t e = 0; e < dh; e++) sc[j] += at(0, b, h, i, e) * at(1, b, h, j, e);
          ok = ok && std::abs(ps[((b * H + h) * S + i) * S + j] - sc[j]) <= 1e-5;
        }
        for (size_t e = 0; e < dh; e++) {
          double c = 0;
          for (size_t j = 0; j < S; j++) c += sc[j] * at(2, b, h, j, e);
          ok = ok && std::abs((merged[b * S + i, h * dh + e]) - c) <= 1e-5;
        }
      }
  CHECK(ok);
}

TEST_CASE("head merge: the product writes the permuted layout, bit-identical") {
  // ctx.permute({0, 2, 1, 3}).view(...) is lowered into the batched
  // product's output strides (no copy kernel); the result must equal the
  // copy of an evaluated ctx bit for bit, including edge tiles.
  const size_t B = 2, S = 70, H = 3, dh = 24, D = H * dh;
  auto qkv = random({B * S, 3 * D});
  auto heads = qkv.view({B, S, 3, H, dh}).permute({2, 0, 3, 1, 4});
  auto q = heads.select(0, 0), k = heads.select(0, 1), v = heads.select(0, 2);
  auto build_ctx = [&] { return (q.batched_dot(k.permute({0, 1, 3, 2})) * 0.125f).batched_dot(v); };
  auto fused = build_ctx().permute({0, 2, 1, 3}).view({B * S, D});
  auto fused2 = build_ctx().permute({0, 2, 1, 3}).view({B * S, D}) * 2.0f;  // into a program
  eval(fused, fused2);
  auto ctx = build_ctx();
  eval(ctx);  // evaluated first: the permute is copied afterwards
  auto plain = ctx.permute({0, 2, 1, 3}).view({B * S, D});
  eval(plain);
  CHECK(fused.shape() == (shape_type{B * S, D}) && plain.shape() == fused.shape());
  const float *a = std::as_const(fused).buffer_data(), *b = std::as_const(plain).buffer_data();
  const float *c = std::as_const(fused2).buffer_data();
  bool same = true, twice = true;
  for (size_t i = 0; i < B * S * D; i++) {
    same = same && std::memcmp(&a[i], &b[i], sizeof(float)) == 0;
    twice = twice && c[i] == b[i] * 2.0f;
  }
  CHECK(same);
  CHECK(twice);
}

TEST_CASE("attention graph runs as one fused launch, matching the unfused graph") {
  // softmax(q k^T * scale) v over head views of a qkv array, the result
  // head-merged: evaluated fused (scores used by nothing else) and unfused
  // (scores requested too), then compared within fp32 rounding.
  const size_t B = 2, S = 77, H = 3, dh = 32, D = H * dh;
  auto qkv = random({B * S, 3 * D});
  auto heads = qkv.view({B, S, 3, H, dh}).permute({2, 0, 3, 1, 4});
  auto q = heads.select(0, 0), k = heads.select(0, 1), v = heads.select(0, 2);
  const float scale = 1.0f / std::sqrt(float(dh));
  auto scores_of = [&] { return q.batched_dot(k.permute({0, 1, 3, 2})) * scale; };
  auto attend = [&](const array<float> &scores) {
    auto attn = scores.view({B * H * S, S}).softmax().view({B, H, S, S});
    return attn.batched_dot(v).permute({0, 2, 1, 3}).view({B * S, D});
  };
  auto fused = attend(scores_of());
  eval(fused);
  auto scores = scores_of();
  auto plain = attend(scores);
  eval(scores, plain);  // the scores are a root: nothing fuses across them
  CHECK(fused.shape() == (shape_type{B * S, D}) && plain.shape() == fused.shape());
  const float *a = std::as_const(fused).buffer_data(), *b = std::as_const(plain).buffer_data();
  float worst = 0.0f;
  for (size_t i = 0; i < B * S * D; i++) worst = std::max(worst, std::abs(a[i] - b[i]));
  CHECK(worst <= 1e-5f);  // v in [0, 1): outputs are convex combinations of v rows
}

TEST_CASE("batched products and attention over more batches than one launch's grid") {
  // 70000 (batch, head) pairs: the library issues them in pieces of at most
  // 65535; fused attention and plain batched_dot match the unfused graph.
  const size_t B = 35000, H = 2, S = 3, dh = 16;
  auto q = random({B, H, S, dh}), k = random({B, H, S, dh}), v = random({B, H, S, dh});
  auto scores_of = [&] { return q.batched_dot(k.permute({0, 1, 3, 2})) * 0.25f; };
  auto attend = [&](const array<float> &scores) {
    return scores.view({B * H * S, S}).softmax().view({B, H, S, S}).batched_dot(v);
  };
  auto fused = attend(scores_of());
  eval(fused);
  auto scores = scores_of();
  auto plain = attend(scores);
  eval(scores, plain);
  float worst = 0.0f;
  for (size_t i = 0; i < B * H * S * dh; i++)
    worst = std::max(worst, std::abs(fused.at(i) - plain.at(i)));
  CHECK(worst <= 1e-5f);
  // the scores themselves against a host dot product (first and last pair)
  for (size_t bh : {size_t(0), B * H - 1}) {
    const size_t b = bh / H, h = bh % H;
    float s = 0.0f;
    for (size_t d = 0; d < dh; d++) s += q.at({b, h, 2, d}) * k.at({b, h, 1, d});
    CHECK(std::abs(scores.at({b, h, 2, 1}) - s * 0.25f) <= 1e-5f);
  }
}

TEST_CASE("conv2d: same padding closed form and the 1x1 kernel as a product") {
  // ones in and ones weights: C_in times the taps inside the image
  auto x = ones<float>({1, 3, 3, 2});
  auto w = ones<float>({1, 3, 3, 2});
  auto y = x.conv2d(w, 3);
  CHECK(y.shape() == (shape_type{1, 3, 3, 1}));
  const float want[9] = {8, 12, 8, 12, 18, 12, 8, 12, 8};
  bool ok = true;
  for (size_t i = 0; i < 9; i++) ok = ok && y.at(i) == want[i];
  CHECK(ok);
  // a 1x1 kernel is the pixels times the weight's transpose
  auto img = random({2, 5, 7, 12}) - 0.5f;
  auto k1 = random({9, 1, 1, 12}) - 0.5f;
  auto conv = img.conv2d(k1, 1);
  auto prod = img.view({70, 12}).dot(k1.view({9, 12}).transpose());
  eval(conv, prod);
  CHECK(conv.shape() == (shape_type{2, 5, 7, 9}));
  float worst = 0.0f;
  for (size_t i = 0; i < 70 * 9; i++) worst = std::max(worst, std::abs(conv.at(i) - prod.at(i)));
  CHECK(worst <= 1e-5f);
  CHECK_THROWS_WITH(img.conv2d(k1, 3), "array: conv2d weight shape does not match the input.");
  CHECK_THROWS_WITH(img.view({70, 12}).conv2d(k1, 1),
                    "array: conv2d requires a 4D NHWC input and a 4D OHWI weight.");
}

TEST_CASE("conv2d inside an eval graph: strided input view, relu and a channel bias after it") {
  // The input is an H <-> W transposed view (strides, no copy) that the
  // lowering makes contiguous; the result feeds a fused elementwise tail.
  const size_t N = 2, H = 5, W = 6, Ci = 4, K = 3, Co = 5;
  auto base = random({N, W, H, Ci}) - 0.5f;
  auto w = random({Co, K, K, Ci}) - 0.5f;
  auto b = random({Co}) - 0.5f;
  eval(base, w, b);
  auto xin = base.permute({0, 2, 1, 3});  // {N, H, W, Ci}
  CHECK(xin.shape() == (shape_type{N, H, W, Ci}));
  auto y = xin.conv2d(w, K).relu() + b;
  eval(y);
  float worst = 0.0f;
  for (size_t n = 0; n < N; n++)
    for (size_t i = 0; i < H; i++)
      for (size_t j = 0; j < W; j++)
        for (size_t o = 0; o < Co; o++) {
          double acc = 0.0;
          for (size_t kh = 0; kh < K; kh++)
            for (size_t kw = 0; kw < K; kw++) {
              const long ih = long(i) + long(kh) - 1, iw = long(j) + long(kw) - 1;
              if (ih < 0 || iw < 0 || ih >= long(H) || iw >= long(W)) continue;
              for (size_t c = 0; c < Ci; c++)
                acc += double(base.at({n, size_t(iw), size_t(ih), c})) * double(w.at({o, kh, kw, c}));
            }
          const double ref = std::max(acc, 0.0) + double(b.at(o));
          worst = std::max(worst, float(std::abs(ref - double(y.at({n, i, j, o})))));
        }
  CHECK(worst <= 1e-5f);
}

TEST_CASE("large arrays round-trip through pinned host mirrors") {
  // 4 MiB: above the size from which host mirrors are pinned
  const size_t n = size_t(1) << 20;
  std::vector<float> v(n);
  for (size_t i = 0; i < n; i++) v[i] = float(i % 1000) * 0.5f;
  auto x = array<float>({n}, v);
  auto y = x * 2.0f;  // uploads x
  eval(y);
  bool ok = true;
  for (size_t i = 0; i < n; i++) ok = ok && y.at(i) == v[i] * 2.0f;  // downloads y
  CHECK(ok);
  x.at(5) = 7.0f;  // host write: the device copy is stale and uploads again
  auto z = x + 1.0f;
  eval(z);
  CHECK(z.at(5) == 8.0f);
  CHECK(z.at(n - 1) == v[n - 1] + 1.0f);
}

HOST_CASE("view, permute and select on evaluated arrays") {
  auto m = array<int>({2, 3, 4}, iota_n(24));
  auto p = m.permute({2, 0, 1});
  CHECK(p.shape() == (shape_type{4, 2, 3}));
  CHECK((p[1, 0, 2]) == (m[0, 2, 1]) && (p[3, 1, 0]) == (m[1, 0, 3]));
  auto s = m.select(1, 2);
  CHECK(s.shape() == (shape_type{2, 4}));
  CHECK(array_equal(s, {{9, 10, 11, 12}, {21, 22, 23, 24}}));
  auto v = m.view({6, 4});
  CHECK(v.shape() == (shape_type{6, 4}) && (v[5, 3]) == 24);
  CHECK_THROWS_WITH(m.view({5, 5}), "array: invalid shape for view.");
  CHECK_THROWS_WITH(m.permute({0, 0, 1}), "array: invalid permutation.");
  CHECK_THROWS_WITH(m.select(1, 3), "array: select is out of bounds.");
}

TEST_CASE("relu of linear runs in the GEMM epilogue") {
  auto x = random({37, 70}) - 0.5f;
  auto W = random({70, 45}) - 0.5f;
  auto b = random({45}) - 0.5f;
  eval(x, W, b);
  auto y = x.linear(W, b).relu();
  auto z = x.linear(W, b);  // unfused twin for the bit-exact comparison
  eval(y, z);
  bool ok = true, some_zero = false, some_pos = false;
  for (size_t i = 0; i < 37; i++)
    for (size_t j = 0; j < 45; j++) {
      const float zv = z[i, j], yv = y[i, j];
      ok = ok && yv == std::max(zv, 0.0f);
      some_zero = some_zero || yv == 0.0f;
      some_pos = some_pos || yv > 0.0f;
    }
  CHECK(ok && some_zero && some_pos);
}

TEST_CASE("products the planner runs on the K-group 64x64 tile: transposed views, linear + relu") {
  // Shapes whose 64 x 64 tiles (times a few K splits) fill the CUs once run
  // with K halved between two wave groups of each workgroup; every operand
  // layout through transposed views, against host double sums on sampled
  // elements with the SGEMM bar 1e-5 * sqrt(K) * sum |a b|.
  auto check = [](const array<float> &c, auto a_at, auto b_at, size_t M, size_t N, size_t K,
                  auto off) {
    bool ok = true;
    for (size_t t = 0; t < 64; t++) {
      const size_t i = (t * 389 + 7) % M, j = (t * 211 + 3) % N;
      double s = off(j), sa = std::abs(off(j));
      for (size_t k = 0; k < K; k++) {
        const double p = double(a_at(i, k)) * double(b_at(k, j));
        s += p;
        sa += std::abs(p);
      }
      ok = ok && std::abs(double(c[i, j]) - s) <= 1e-5 * std::sqrt(double(K)) * sa + 1e-30;
    }
    return ok;
  };
  int n = 0, tiles[2] = {0, 0}, splits[2] = {0, 0}, rows[2] = {0, 0};
  for (auto [M, N, K] : {std::tuple<size_t, size_t, size_t>{1024, 1024, 1024}, {256, 2048, 512}}) {
    auto a = random({M, K}) - 0.5f, at = random({K, M}) - 0.5f;
    auto b = random({K, N}) - 0.5f, bt = random({N, K}) - 0.5f;
    eval(a, at, b, bt);
    auto nn = a.dot(b), tn = at.transpose().dot(b), nt = a.dot(bt.transpose()),
         tt = at.transpose().dot(bt.transpose());
    eval(nn, tn, nt, tt);
    silgpu_gemm_last_plan(&n, tiles, splits, rows);
    CHECK(n == 1);
    CHECK(tiles[0] == 9);
    auto none = [](size_t) { return 0.0; };
    CHECK(check(nn, [&](size_t i, size_t k) { return a[i, k]; },
                [&](size_t k, size_t j) { return b[k, j]; }, M, N, K, none));
    CHECK(check(tn, [&](size_t i, size_t k) { return at[k, i]; },
                [&](size_t k, size_t j) { return b[k, j]; }, M, N, K, none));
    CHECK(check(nt, [&](size_t i, size_t k) { return a[i, k]; },
                [&](size_t k, size_t j) { return bt[j, k]; }, M, N, K, none));
    CHECK(check(tt, [&](size_t i, size_t k) { return at[k, i]; },
                [&](size_t k, size_t j) { return bt[j, k]; }, M, N, K, none));
  }
  // linear + relu at 128 x 2048 x 768 (4 K splits on the K-group tile),
  // bit-identical to relu applied to the unfused twin
  auto x = random({128, 768}) - 0.5f;
  auto W = random({768, 2048}) - 0.5f;
  auto bias = random({2048}) - 0.5f;
  eval(x, W, bias);
  auto y = x.linear(W, bias).relu();
  eval(y);
  silgpu_gemm_last_plan(&n, tiles, splits, rows);
  CHECK(n == 1);
  CHECK(tiles[0] == 9);
  auto z = x.linear(W, bias);
  eval(z);
  bool ok = true;
  for (size_t i = 0; i < 128; i++)
    for (size_t j = 0; j < 2048; j++) ok = ok && y[i, j] == std::max(z[i, j], 0.0f);
  CHECK(ok);
  CHECK(check(z, [&](size_t i, size_t k) { return x[i, k]; },
              [&](size_t k, size_t j) { return W[k, j]; }, 128, 2048, 768,
              [&](size_t j) { return double(bias.at(j)); }));
}

//------------------------------------------------------------------------------
// GPU: storage boundary (the reference's msl:: tests, test/test_array.cpp:643-706)
//------------------------------------------------------------------------------

TEST_CASE("msl add float / int / broadcast on raw storage") {
  auto a = storage::make(4 * sizeof(float));
  auto b = storage::make(4 * sizeof(float));
  auto o = storage::make(4 * sizeof(float));
  float av[] = {1, 2, 3, 4}, bv[] = {10, 20, 30, 40};
  std::memcpy(a.data, av, sizeof(av));
  std::memcpy(b.data, bv, sizeof(bv));
  a.len = b.len = o.len = 4;
  msl::add<float>(a, b, o);
  synchronize();
  CHECK(array_equal(array<float>({4}, static_cast<float *>(o.data)), {11.0f, 22.0f, 33.0f, 44.0f}));

  auto ia = storage::make(4 * sizeof(int)), ib = storage::make(4 * sizeof(int)),
       io = storage::make(4 * sizeof(int));
  int iav[] = {1, 2, 3, 4}, ibv[] = {10, 20, 30, 40};
  std::memcpy(ia.data, iav, sizeof(iav));
  std::memcpy(ib.data, ibv, sizeof(ibv));
  ia.len = ib.len = io.len = 4;
  msl::add<int>(ia, ib, io);
  synchronize();
  CHECK(array_equal(array<int>({4}, static_cast<int *>(io.data)), {11, 22, 33, 44}));

  auto s1 = storage::make(sizeof(float));
  float one[] = {10.0f};
  std::memcpy(s1.data, one, sizeof(one));
  s1.len = 1;
  msl::add<float>(a, s1, o);
  synchronize();
  CHECK(array_equal(array<float>({4}, static_cast<float *>(o.data)), {11.0f, 12.0f, 13.0f, 14.0f}));
}

TEST_CASE("raw storage rewritten through data after a kernel read is uploaded again") {
  // The reference's unified-memory contract: the host writes `data` directly
  // between launches, with no call that tells the storage.
  auto a = storage::make(4 * sizeof(float));
  auto b = storage::make(4 * sizeof(float));
  auto o = storage::make(4 * sizeof(float));
  a.len = b.len = o.len = 4;
  const float av[] = {1, 2, 3, 4}, bv[] = {10, 20, 30, 40}, av2[] = {5, 6, 7, 8};
  std::memcpy(a.data, av, sizeof(av));
  std::memcpy(b.data, bv, sizeof(bv));
  msl::add<float>(a, b, o);
  synchronize();
  CHECK(array_equal(array<float>({4}, static_cast<float *>(o.data)), {11.0f, 22.0f, 33.0f, 44.0f}));
  std::memcpy(a.data, av2, sizeof(av2));
  msl::add<float>(a, b, o);
  synchronize();
  CHECK(array_equal(array<float>({4}, static_cast<float *>(o.data)), {15.0f, 26.0f, 37.0f, 48.0f}));
  // the output of the last call used as an input after its host copy changed
  static_cast<float *>(o.data)[0] = 100.0f;
  msl::add<float>(o, b, a);
  synchronize();
  CHECK(array_equal(array<float>({4}, static_cast<float *>(a.data)), {110.0f, 46.0f, 67.0f, 88.0f}));
}

TEST_CASE("in-place kernels on a fresh raw storage read the host data") {
  // Input and output are the same storage: the pending upload must happen
  // before the output is marked device-written.
  auto x = storage::make(3 * sizeof(float));
  x.len = 3;
  const float xv[] = {0.0f, 1.0f, -1.0f};
  std::memcpy(x.data, xv, sizeof(xv));
  msl::sigmoid(x, x);
  synchronize();
  const float *r = static_cast<const float *>(x.data);
  CHECK(is_close(r[0], 0.5f, 1e-6f) && is_close(r[1], 0.7310586f, 1e-6f) &&
        is_close(r[2], 0.2689414f, 1e-6f));
  auto y = storage::make(4 * sizeof(float));
  y.len = 4;
  const float yv[] = {1, 2, 3, 4};
  std::memcpy(y.data, yv, sizeof(yv));
  msl::mul<float>(y, y, y);
  synchronize();
  CHECK(array_equal(array<float>({4}, static_cast<float *>(y.data)), {1.0f, 4.0f, 9.0f, 16.0f}));
}

TEST_CASE("slice and row views of a device array feed linear, sum(0) and dot") {
  // Zero-copy views (the reference's slice, include/array.h:1177-1187, as
  // its MNIST benchmark uses it for batches) of an evaluated device array,
  // against float64 sums of the same host values.
  const size_t R = 64, K = 96, N = 40, r0 = 10, rn = 33;
  auto X = random({R, K}) - 0.5f;
  auto W = random({K, N}) - 0.5f;
  auto b = random({N}) - 0.5f;
  eval(X, W, b);
  auto Xs = X.slice(r0, rn);
  CHECK(Xs.shape() == (shape_type{rn, K}));
  CHECK(std::as_const(Xs).buffer_data() == std::as_const(X).buffer_data() + r0 * K);
  auto row = X[r0 + 7];  // a row view: a 1-D vector times a matrix (the GEMV path)
  auto Y = Xs.linear(W, b);
  auto S = Xs.sum(0);
  auto yr = row.dot(W);
  eval(Y, S, yr);
  CHECK(Y.shape() == (shape_type{rn, N}) && S.shape() == shape_type{K} && yr.shape() == shape_type{N});
  const float tol = 1e-5f * std::sqrt(float(K));
  bool ok = true;
  for (size_t i = 0; i < rn; i++)
    for (size_t j = 0; j < N; j++) {
      double acc = 0.0, mag = 0.0;
      for (size_t k = 0; k < K; k++) {
        const double t = double(X[r0 + i, k]) * double(W[k, j]);
        acc += t;
        mag += std::abs(t);
      }
      acc += double(b.at(j));
      mag += std::abs(double(b.at(j)));
      ok = ok && std::abs(double(Y[i, j]) - acc) <= tol * mag + 1e-30;
    }
  CHECK(ok);
  bool sok = true;
  for (size_t k = 0; k < K; k++) {
    double acc = 0.0, mag = 0.0;
    for (size_t i = 0; i < rn; i++) {
      acc += double(X[r0 + i, k]);
      mag += std::abs(double(X[r0 + i, k]));
    }
    sok = sok && std::abs(double(S.at(k)) - acc) <= 1e-5 * std::abs(acc) + 6e-8 * mag + 1e-30;
  }
  CHECK(sok);
  bool rok = true;
  for (size_t j = 0; j < N; j++) {
    double acc = 0.0, mag = 0.0;
    for (size_t k = 0; k < K; k++) {
      const double t = double(X[r0 + 7, k]) * double(W[k, j]);
      acc += t;
      mag += std::abs(t);
    }
    rok = rok && std::abs(double(yr.at(j)) - acc) <= tol * mag + 1e-30;
  }
  CHECK(rok);
}

TEST_CASE("host writes after device use are uploaded") {
  auto x = ones<float>({8192});
  auto s1 = x.sum();
  x.at(5) = 3.0f;  // host write marks the device copy stale
  auto s2 = x.sum();
  CHECK(s1 == 8192.0f && s2 == 8194.0f);
}

// The reference's two-layer network on XOR (test/test_2lnn.cpp:5-140), with a
// fixed initialisation in place of sil::random.  A float32 numpy run of the
// same 2000 epochs from this start reaches outputs {0.027, 0.971, 0.971,
// 0.034} and loss 8.9e-4.
TEST_CASE("2 layer NN learns xor (forward, sigmoid_backward, transposed dot, -=)") {
  auto W1 = array<float>{{0.9f, -0.8f, 0.4f}, {0.7f, -0.9f, -0.5f}};
  auto b1 = array<float>{-0.3f, 0.4f, 0.2f};
  auto W2 = array<float>({3, 1}, std::vector<float>{0.8f, -0.7f, 0.5f});
  auto b2 = array<float>{0.2f};
  const auto X = array<float>{{0, 0}, {0, 1}, {1, 0}, {1, 1}};
  const auto Y = array<float>{{0}, {1}, {1}, {0}};
  const float lr = 0.5f;
  float loss = 0.0f;
  array<float> out;
  for (int epoch = 0; epoch < 2000; epoch++) {
    auto net1 = X.linear(W1, b1);
    auto out1 = net1.sigmoid();
    auto net2 = out1.linear(W2, b2);
    out = net2.sigmoid();
    loss = out.mean_square_error(Y);
    auto dout = 1.0f * (2 * (out - Y));
    dout = net2.sigmoid_backward(dout);
    auto dout1 = dout.dot(W2.transpose());
    auto dW2 = out1.transpose().dot(dout);
    auto db2 = dout.sum(0);
    dout = net1.sigmoid_backward(dout1);
    auto dW1 = X.transpose().dot(dout);
    auto db1 = dout.sum(0);
    W1 -= dW1 * lr;
    b1 -= db1 * lr;
    W2 -= dW2 * lr;
    b2 -= db2 * lr;
  }
  CHECK(loss < 2e-3f);
  const float expect[] = {0.027f, 0.971f, 0.971f, 0.034f};
  for (size_t i = 0; i < 4; i++) CHECK(is_close((out[i, 0]), expect[i], 5e-3f));
  CHECK(array_equal(where<float>(out > 0.5f, 1, 0), {{0}, {1}, {1}, {0}}));
}

int main(int argc, char **argv) { return harness::run(argc, argv); }
