// C++ front-end test: seeded random sil::eval graphs against a float64 host
// shadow.  Each graph starts from a random [R, C] input (R, C up to 1100) and
// applies 3-14 random nodes over a pool of shared operands: elementwise ops
// with numpy broadcasting (a row, a column, a scalar), scalar affine nodes,
// relu, sigmoid, sigmoid_backward, pow, compound assignment, dot with the
// reference's 1-D promotion and transposed views (include/array.h:1376-1403,
// 2658-2688; {1, n} transposes to {n} and {n} to {1, n}, :1051-1099),
// linear, linear_sigmoid, relu(linear), residual adds, a product times a
// scalar, softmax, layer_norm, sum(axis), slice, 3-D views with permute,
// select and batched_dot, an attention graph with its head merge
// (bench/composite/bench_transformer.cpp:55-68 batched), conv2d, and scalar
// reductions and argmax taken mid-graph (which evaluate part of the graph
// early), and host writes into evaluated arrays (directly and through row
// views) that later device nodes read.  Four roots per graph are evaluated in one sil::eval and each is
// compared with the shadow: |got - ref| <= 1e-3 (rms(ref) + |ref|) + 1e-6, a
// bar loose enough for fp32 rounding through a chain of nodes and tight
// enough for a wrong fusion, operand, index or broadcast, which err by O(1).
// Usage: random_graphs SEED GRAPHS; prints "N graphs, F failures".
#include <silarray.h>

#include <cstdlib>
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <functional>
#include <random>
#include <string>
#include <vector>

using namespace sil;

using Arr = array<float>;

struct H {
  std::vector<size_t> shape;
  std::vector<double> v;
  size_t rows() const { return shape.size() == 2 ? shape[0] : 1; }
  size_t cols() const { return shape.empty() ? 1 : shape.back(); }
};

struct Val {
  Arr a;
  H h;
  std::string desc;
};

static std::mt19937_64 rng_;
static size_t g_fails = 0;  // mismatches found inside step()
static double unif(double lo, double hi) { return std::uniform_real_distribution<double>(lo, hi)(rng_); }
static size_t irand(size_t lo, size_t hi) { return std::uniform_int_distribution<size_t>(lo, hi)(rng_); }

static Val fresh(std::vector<size_t> shape, double lo, double hi) {
  size_t n = 1;
  for (auto s : shape) n *= s;
  std::vector<float> f(n);
  H h{shape, std::vector<double>(n)};
  for (size_t i = 0; i < n; i++) {
    f[i] = static_cast<float>(unif(lo, hi));
    h.v[i] = f[i];
  }
  shape_type sh(shape.begin(), shape.end());
  return {Arr(sh, f), h, "in" + std::to_string(n)};
}

// numpy broadcasting for ranks <= 2
static H bcast(const H &x, const H &y, const std::function<double(double, double)> &f) {
  size_t nd = std::max(x.shape.size(), y.shape.size());
  std::vector<size_t> xs(nd, 1), ys(nd, 1), os(nd);
  for (size_t i = 0; i < x.shape.size(); i++) xs[nd - x.shape.size() + i] = x.shape[i];
  for (size_t i = 0; i < y.shape.size(); i++) ys[nd - y.shape.size() + i] = y.shape[i];
  for (size_t d = 0; d < nd; d++) os[d] = std::max(xs[d], ys[d]);
  H o{os, {}};
  size_t n = 1;
  for (auto s : os) n *= s;
  o.v.resize(n);
  for (size_t i = 0; i < n; i++) {
    size_t rem = i, xi = 0, yi = 0, xst = 1, yst = 1;
    for (size_t d = nd; d-- > 0;) {
      size_t c = rem % os[d];
      rem /= os[d];
      xi += (xs[d] == 1 ? 0 : c) * xst;
      yi += (ys[d] == 1 ? 0 : c) * yst;
      xst *= xs[d];
      yst *= ys[d];
    }
    o.v[i] = f(x.v[xi], y.v[yi]);
  }
  return o;
}

static H dot(const H &x, const H &y) {  // 1-D promotion as numpy
  bool xv = x.shape.size() == 1, yv = y.shape.size() == 1;
  if (x.shape.empty() || y.shape.empty() || x.shape.size() > 2 || y.shape.size() > 2 ||
      x.shape.back() != y.shape[0])
    throw std::runtime_error("shadow: invalid dot " + std::to_string(x.shape.size()) + "-D x " +
                             std::to_string(y.shape.size()) + "-D");
  size_t M = xv ? 1 : x.shape[0], K = x.shape.back(), N = yv ? 1 : y.shape[1];
  H o;
  if (xv && yv) o.shape = {};
  else if (xv) o.shape = {N};
  else if (yv) o.shape = {M};
  else o.shape = {M, N};
  o.v.assign(M * N, 0.0);
  for (size_t m = 0; m < M; m++)
    for (size_t k = 0; k < K; k++) {
      double a = x.v[m * K + k];
      for (size_t n = 0; n < N; n++) o.v[m * N + n] += a * y.v[yv ? k : k * N + n];
    }
  return o;
}

static H transpose(const H &x) {
  // the reference's transpose: {n} -> {1, n}, {1, n} -> {n}, 2-D swap
  if (x.shape.size() == 1) return H{{1, x.shape[0]}, x.v};
  if (x.shape[0] == 1) return H{{x.shape[1]}, x.v};
  H o{{x.shape[1], x.shape[0]}, std::vector<double>(x.v.size())};
  for (size_t r = 0; r < x.shape[0]; r++)
    for (size_t c = 0; c < x.shape[1]; c++) o.v[c * x.shape[0] + r] = x.v[r * x.shape[1] + c];
  return o;
}

static H unary(const H &x, const std::function<double(double)> &f) {
  H o = x;
  for (auto &e : o.v) e = f(e);
  return o;
}

static H softmax(const H &x) {
  H o = x;
  size_t R = x.rows(), C = x.cols();
  for (size_t r = 0; r < R; r++) {
    double m = -INFINITY, s = 0;
    for (size_t c = 0; c < C; c++) m = std::max(m, x.v[r * C + c]);
    for (size_t c = 0; c < C; c++) s += std::exp(x.v[r * C + c] - m);
    for (size_t c = 0; c < C; c++) o.v[r * C + c] = std::exp(x.v[r * C + c] - m) / s;
  }
  return o;
}

static H layer_norm(const H &x, const H &g, const H &b) {
  H o = x;
  size_t R = x.rows(), C = x.cols();
  for (size_t r = 0; r < R; r++) {
    double mu = 0, ss = 0;
    for (size_t c = 0; c < C; c++) mu += x.v[r * C + c];
    mu /= C;
    for (size_t c = 0; c < C; c++) ss += (x.v[r * C + c] - mu) * (x.v[r * C + c] - mu);
    double inv = 1.0 / std::sqrt(ss / C + 1e-5);
    for (size_t c = 0; c < C; c++) o.v[r * C + c] = (x.v[r * C + c] - mu) * inv * g.v[c] + b.v[c];
  }
  return o;
}

static H sum_axis(const H &x, size_t ax) {
  size_t R = x.shape[0], C = x.shape[1];
  H o;
  o.shape = {ax == 0 ? C : R};
  o.v.assign(o.shape[0], 0.0);
  for (size_t r = 0; r < R; r++)
    for (size_t c = 0; c < C; c++) o.v[ax == 0 ? c : r] += x.v[r * C + c];
  return o;
}

static size_t count(const std::vector<size_t> &s) {
  size_t n = 1;
  for (auto e : s) n *= e;
  return n;
}
static H permute(const H &x, const std::vector<size_t> &ax) {
  const size_t nd = x.shape.size();
  H o;
  o.shape.resize(nd);
  for (size_t i = 0; i < nd; i++) o.shape[i] = x.shape[ax[i]];
  o.v.resize(x.v.size());
  std::vector<size_t> xst(nd, 1);
  for (size_t d = nd - 1; d-- > 0;) xst[d] = xst[d + 1] * x.shape[d + 1];
  for (size_t i = 0; i < o.v.size(); i++) {
    size_t r = i, off = 0;
    for (size_t d = nd; d-- > 0;) {
      size_t c = r % o.shape[d];
      r /= o.shape[d];
      off += c * xst[ax[d]];
    }
    o.v[i] = x.v[off];
  }
  return o;
}
static H select(const H &x, size_t axis, size_t idx) {
  H o;
  o.shape = x.shape;
  o.shape.erase(o.shape.begin() + axis);
  size_t outer = count(std::vector<size_t>(x.shape.begin(), x.shape.begin() + axis));
  size_t inner = count(std::vector<size_t>(x.shape.begin() + axis + 1, x.shape.end()));
  for (size_t a = 0; a < outer; a++)
    for (size_t i = 0; i < inner; i++) o.v.push_back(x.v[(a * x.shape[axis] + idx) * inner + i]);
  return o;
}
static H sum_any(const H &x, size_t axis) {
  H o;
  o.shape = x.shape;
  o.shape.erase(o.shape.begin() + axis);
  size_t outer = count(std::vector<size_t>(x.shape.begin(), x.shape.begin() + axis));
  size_t inner = count(std::vector<size_t>(x.shape.begin() + axis + 1, x.shape.end()));
  o.v.assign(outer * inner, 0.0);
  for (size_t a = 0; a < outer; a++)
    for (size_t k = 0; k < x.shape[axis]; k++)
      for (size_t i = 0; i < inner; i++) o.v[a * inner + i] += x.v[(a * x.shape[axis] + k) * inner + i];
  return o;
}
static size_t divisor(size_t n) {  // a random divisor of n
  std::vector<size_t> d;
  for (size_t i = 1; i <= n; i++)
    if (n % i == 0) d.push_back(i);
  return d[irand(0, d.size() - 1)];
}

static std::string shp(const H &h) {
  std::string s = "{";
  for (size_t i = 0; i < h.shape.size(); i++) s += (i ? "," : "") + std::to_string(h.shape[i]);
  return s + "}";
}

// One random op on the pool; returns false if it could not apply.
static bool step(std::vector<Val> &pool) {
  Val &x = pool[irand(pool.size() > 4 ? pool.size() - 4 : 0, pool.size() - 1)];
  Val &y = pool[irand(0, pool.size() - 1)];
  const size_t nd = x.h.shape.size();
  switch (irand(0, 29)) {
    case 0: {  // binary with a broadcast-compatible partner
      int op = static_cast<int>(irand(0, 3));
      std::vector<size_t> ps;
      switch (irand(0, 3)) {
        case 0: ps = x.h.shape; break;
        case 1: ps = {x.h.cols()}; break;
        case 2: if (nd == 2) { ps = {x.h.shape[0], 1}; break; } ps = x.h.shape; break;
        default: ps = nd == 2 ? std::vector<size_t>{1, x.h.cols()} : x.h.shape;
      }
      Val p = fresh(ps, op == 3 ? 0.5 : -1.0, op == 3 ? 2.0 : 1.0);
      bool swap = op != 3 && irand(0, 1);
      const Val &l = swap ? p : x, &r = swap ? x : p;
      static const char *nm[] = {"+", "-", "*", "/"};
      std::function<double(double, double)> f[] = {
          [](double a, double b) { return a + b; }, [](double a, double b) { return a - b; },
          [](double a, double b) { return a * b; }, [](double a, double b) { return a / b; }};
      Arr res = op == 0 ? l.a + r.a : op == 1 ? l.a - r.a : op == 2 ? l.a * r.a : l.a / r.a;
      pool.push_back({res, bcast(l.h, r.h, f[op]), "(" + l.desc + nm[op] + r.desc + ")"});
      return true;
    }
    case 1: {  // same-shape binary between pool values
      if (x.h.shape != y.h.shape) return false;
      bool add = irand(0, 1);
      pool.push_back({add ? x.a + y.a : x.a * y.a,
                      bcast(x.h, y.h, add ? std::function<double(double, double)>([](double a, double b) { return a + b; })
                                          : std::function<double(double, double)>([](double a, double b) { return a * b; })),
                      std::string(add ? "add" : "mul") + shp(x.h)});
      return true;
    }
    case 2: {  // scalar affine chain
      float a = static_cast<float>(unif(0.5, 1.5)), b = static_cast<float>(unif(-1, 1));
      int k = static_cast<int>(irand(0, 2));
      Arr res = k == 0 ? x.a * a + b : k == 1 ? b - x.a * a : (x.a + b) * a;
      double da = a, db = b;
      H h = unary(x.h, [&](double v) { return k == 0 ? v * da + db : k == 1 ? db - v * da : (v + db) * da; });
      pool.push_back({res, h, "aff" + shp(x.h)});
      return true;
    }
    case 3:
      pool.push_back({x.a.relu(), unary(x.h, [](double v) { return v > 0 ? v : 0.0; }), "relu"});
      return true;
    case 4:
      pool.push_back({x.a.sigmoid(), unary(x.h, [](double v) { return 1 / (1 + std::exp(-v)); }), "sig"});
      return true;
    case 5: {  // dot with a fresh right operand (1-D promotion included)
      size_t K = x.h.cols(), N = irand(1, 300);
      bool vec = irand(0, 4) == 0;
      Val w = fresh(vec ? std::vector<size_t>{K} : std::vector<size_t>{K, N}, -1.0 / std::sqrt(K), 1.0 / std::sqrt(K));
      pool.push_back({x.a.dot(w.a), dot(x.h, w.h), "dot" + shp(x.h) + shp(w.h)});
      if (pool.back().h.shape.empty()) { pool.pop_back(); return false; }
      return true;
    }
    case 6: {  // dot with a transposed view on either side
      if (nd != 2) return false;
      size_t R = x.h.shape[0], C = x.h.shape[1], N = irand(1, 200);
      H hr;
      if (irand(0, 1)) {  // x^T . w : [C, R] . [R, N]
        Val w = fresh({R, N}, -1.0 / std::sqrt(R), 1.0 / std::sqrt(R));
        try { hr = dot(transpose(x.h), w.h); } catch (const std::exception &) { return false; }
        if (hr.shape.empty()) return false;
        pool.push_back({x.a.transpose().dot(w.a), hr, "dotT"});
      } else {  // x . w^T : [R, C] . ([N, C])^T
        Val w = fresh({N, C}, -1.0 / std::sqrt(C), 1.0 / std::sqrt(C));
        try { hr = dot(x.h, transpose(w.h)); } catch (const std::exception &) { return false; }
        if (hr.shape.empty()) return false;
        pool.push_back({x.a.dot(w.a.transpose()), hr, "dotWT"});
      }
      return true;
    }
    case 7: {  // linear / linear_sigmoid
      if (nd != 2) return false;
      size_t K = x.h.cols(), N = irand(1, 300);
      Val w = fresh({K, N}, -1.0 / std::sqrt(K), 1.0 / std::sqrt(K));
      Val b = fresh({N}, -0.5, 0.5);
      H h = bcast(dot(x.h, w.h), b.h, [](double p, double q) { return p + q; });
      if (irand(0, 1)) {
        pool.push_back({x.a.linear_sigmoid(w.a, b.a), unary(h, [](double v) { return 1 / (1 + std::exp(-v)); }), "linsig"});
      } else {
        pool.push_back({x.a.linear(w.a, b.a), h, "lin"});
      }
      return true;
    }
    case 8:
      if (nd != 2) return false;
      pool.push_back({x.a.softmax(), softmax(x.h), "softmax" + shp(x.h)});
      return true;
    case 9: {
      if (nd != 2) return false;
      Val g = fresh({x.h.cols()}, 0.5, 1.5), b = fresh({x.h.cols()}, -1, 1);
      pool.push_back({x.a.layer_norm(g.a, b.a), layer_norm(x.h, g.h, b.h), "ln" + shp(x.h)});
      return true;
    }
    case 10: {
      if (nd != 2) return false;
      size_t ax = irand(0, 1);
      pool.push_back({x.a.sum(ax), sum_axis(x.h, ax), "sum" + std::to_string(ax)});
      return true;
    }
    case 11:
      if (nd != 2) return false;
      pool.push_back({x.a.transpose(), transpose(x.h), "T"});
      return true;
    case 12: {  // slice of rows
      if (nd != 2 || x.h.shape[0] < 2) return false;
      size_t st = irand(0, x.h.shape[0] - 1), cnt = irand(1, x.h.shape[0] - st);
      H h{{cnt, x.h.shape[1]}, std::vector<double>(x.h.v.begin() + st * x.h.shape[1],
                                                   x.h.v.begin() + (st + cnt) * x.h.shape[1])};
      pool.push_back({x.a.slice(st, cnt), h, "slice"});
      return true;
    }
    case 14: {  // attention graph on fresh q, k, v, head-merged to 2-D
      size_t B = irand(1, 2), Hh = irand(1, 3), S = irand(1, 70), Dd = irand(0, 3) == 0 ? irand(1, 40) : 16 << irand(0, 2);
      Val q = fresh({B, Hh, S, Dd}, -1, 1), k = fresh({B, Hh, S, Dd}, -1, 1), v = fresh({B, Hh, S, Dd}, -1, 1);
      float scale = 1.0f / std::sqrt(float(Dd));
      auto scores = q.a.batched_dot(k.a.permute({0, 1, 3, 2})) * scale;
      auto attn = scores.view({B * Hh * S, S}).softmax().view({B, Hh, S, S});
      auto ctx = attn.batched_dot(v.a);
      auto merged = ctx.permute({0, 2, 1, 3}).view({B * S, Hh * Dd});
      H h{{B * S, Hh * Dd}, std::vector<double>(B * S * Hh * Dd)};
      std::vector<double> sc(S);
      for (size_t b = 0; b < B; b++)
        for (size_t hh = 0; hh < Hh; hh++)
          for (size_t i = 0; i < S; i++) {
            const size_t base = (b * Hh + hh) * S;
            double m = -INFINITY, sum = 0;
            for (size_t j = 0; j < S; j++) {
              double acc = 0;
              for (size_t d = 0; d < Dd; d++) acc += q.h.v[(base + i) * Dd + d] * k.h.v[(base + j) * Dd + d];
              sc[j] = acc * double(scale);
              m = std::max(m, sc[j]);
            }
            for (size_t j = 0; j < S; j++) { sc[j] = std::exp(sc[j] - m); sum += sc[j]; }
            for (size_t d = 0; d < Dd; d++) {
              double acc = 0;
              for (size_t j = 0; j < S; j++) acc += sc[j] * v.h.v[(base + j) * Dd + d];
              h.v[(b * S + i) * (Hh * Dd) + hh * Dd + d] = acc / sum;
            }
          }
      pool.push_back({merged, h, "attn B" + std::to_string(B) + " H" + std::to_string(Hh) + " S" + std::to_string(S) + " D" + std::to_string(Dd)});
      return true;
    }
    case 15: {  // conv2d on a fresh NHWC input, viewed as [pixels, C_out]
      size_t N = irand(1, 2), Hh = irand(1, 12), W = irand(1, 12), Ci = irand(1, 40), K = irand(1, 5), Co = irand(1, 60);
      Val in = fresh({N, Hh, W, Ci}, -1, 1), w = fresh({Co, K, K, Ci}, -0.3, 0.3);
      H h{{N * Hh * W, Co}, std::vector<double>(N * Hh * W * Co, 0.0)};
      const long pd = long(K / 2);
      for (size_t n = 0; n < N; n++)
        for (size_t y = 0; y < Hh; y++)
          for (size_t xx = 0; xx < W; xx++)
            for (size_t co = 0; co < Co; co++) {
              double acc = 0;
              for (size_t kh = 0; kh < K; kh++)
                for (size_t kw = 0; kw < K; kw++) {
                  long iy = long(y + kh) - pd, ix = long(xx + kw) - pd;
                  if (iy < 0 || iy >= long(Hh) || ix < 0 || ix >= long(W)) continue;
                  for (size_t ci = 0; ci < Ci; ci++)
                    acc += in.h.v[((n * Hh + iy) * W + ix) * Ci + ci] * w.h.v[((co * K + kh) * K + kw) * Ci + ci];
                }
              h.v[((n * Hh + y) * W + xx) * Co + co] = acc;
            }
      pool.push_back({in.a.conv2d(w.a, K).view({N * Hh * W, Co}), h, "conv"});
      return true;
    }
    case 16: {  // scalar reductions: force evaluation mid-graph, compared at once
      double s64 = 0, mn = INFINITY, mx = -INFINITY, sabs = 0;
      for (double e : x.h.v) { s64 += e; sabs += std::fabs(e); mn = std::min(mn, e); mx = std::max(mx, e); }
      float s = x.a.sum(), a = x.a.min(), b = x.a.max();
      double rms = std::sqrt(sabs * sabs / std::max<size_t>(x.h.v.size(), 1)) / std::sqrt(double(std::max<size_t>(x.h.v.size(), 1)));
      if (std::fabs(s - s64) > 1e-4 * sabs + 1e-6 || std::fabs(a - mn) > 1e-3 * (std::fabs(mn) + rms) + 1e-6 ||
          std::fabs(b - mx) > 1e-3 * (std::fabs(mx) + rms) + 1e-6) {
        printf("FAIL scalar reductions of %s %s: %g %g %g vs %g %g %g\n", x.desc.substr(0, 80).c_str(), shp(x.h).c_str(), s, a, b, s64, mn, mx);
        fflush(stdout);
        g_fails++;
      }
      return false;
    }
    case 17: {  // argmax per row, compared at once (ties: shadow may differ by rounding, so only check the value)
      if (nd != 2) return false;
      auto am = x.a.argmax();
      for (size_t r = 0; r < x.h.shape[0]; r++) {
        size_t c = size_t(am.at(r));
        double best = -INFINITY;
        for (size_t j = 0; j < x.h.shape[1]; j++) best = std::max(best, x.h.v[r * x.h.shape[1] + j]);
        if (c >= x.h.shape[1] || std::fabs(x.h.v[r * x.h.shape[1] + c] - best) > 1e-3 * (std::fabs(best) + 1e-2)) {
          printf("FAIL argmax row %zu of %s: col %zu\n", r, shp(x.h).c_str(), c);
          fflush(stdout);
          g_fails++;
          break;
        }
      }
      return false;
    }
    case 18: {  // compound assignment on a copy
      Val p = fresh(x.h.shape, 0.5, 2.0);
      Arr y2 = x.a;
      int k = int(irand(0, 3));
      if (k == 0) y2 += p.a; else if (k == 1) y2 -= p.a; else if (k == 2) y2 *= p.a; else y2 /= p.a;
      std::function<double(double, double)> f[] = {
          [](double a, double b) { return a + b; }, [](double a, double b) { return a - b; },
          [](double a, double b) { return a * b; }, [](double a, double b) { return a / b; }};
      pool.push_back({y2, bcast(x.h, p.h, f[k]), "compound"});
      return true;
    }
    case 19: {  // pow with a positive base
      Val base = fresh(x.h.shape, 0.5, 2.0), e = fresh(x.h.shape, -2.0, 2.0);
      pool.push_back({base.a.pow(e.a), bcast(base.h, e.h, [](double a, double b) { return std::pow(a, b); }), "pow"});
      return true;
    }
    case 20: {  // sigmoid_backward
      Val d = fresh(x.h.shape, -1, 1);
      H h = x.h;
      for (size_t i = 0; i < h.v.size(); i++) {
        double sg = 1 / (1 + std::exp(-x.h.v[i]));
        h.v[i] = d.h.v[i] * sg * (1 - sg);
      }
      pool.push_back({x.a.sigmoid_backward(d.a), h, "sigbwd"});
      return true;
    }
    case 21: {  // product with a scalar on either side (folded into the epilogue)
      if (nd != 2) return false;
      size_t K = x.h.cols(), N = irand(1, 200);
      Val w = fresh({K, N}, -1.0 / std::sqrt(K), 1.0 / std::sqrt(K));
      H p = dot(x.h, w.h);
      float c = float(unif(0.5, 2.0));
      int k = int(irand(0, 3));
      Arr pa = x.a.dot(w.a);
      Arr r = k == 0 ? pa * c : k == 1 ? c - pa : k == 2 ? pa / c : c + pa;
      double cd = c;
      H h = unary(p, [&](double v) { return k == 0 ? v * cd : k == 1 ? cd - v : k == 2 ? v / cd : cd + v; });
      pool.push_back({r, h, "dotscal" + std::to_string(k)});
      return true;
    }
    case 22: {  // relu(linear)
      if (nd != 2) return false;
      size_t K = x.h.cols(), N = irand(1, 300);
      Val w = fresh({K, N}, -1.0 / std::sqrt(K), 1.0 / std::sqrt(K)), b = fresh({N}, -0.5, 0.5);
      H h = bcast(dot(x.h, w.h), b.h, [](double p, double q) { return p + q; });
      pool.push_back({x.a.linear(w.a, b.a).relu(), unary(h, [](double v) { return v > 0 ? v : 0.0; }), "linrelu"});
      return true;
    }
    case 23: {  // x + linear(x) (residual into the epilogue), either side
      if (nd != 2 || x.h.cols() > 2048) return false;
      size_t C = x.h.cols();
      Val w = fresh({C, C}, -1.0 / std::sqrt(C), 1.0 / std::sqrt(C)), b = fresh({C}, -0.5, 0.5);
      H h = bcast(x.h, bcast(dot(x.h, w.h), b.h, [](double p, double q) { return p + q; }), [](double p, double q) { return p + q; });
      Arr l = x.a.linear(w.a, b.a);
      pool.push_back({irand(0, 1) ? x.a + l : l + x.a, h, "linresid"});
      return true;
    }
    case 24: {  // 3-D detour: view, permute, broadcast op, reduce or view back
      if (nd != 2 || x.h.shape[0] < 2) return false;
      size_t R = x.h.shape[0], C = x.h.shape[1], a = divisor(R), b = R / a;
      std::vector<size_t> sh3{a, b, C};
      std::vector<std::vector<size_t>> perms{{0, 1, 2}, {0, 2, 1}, {1, 0, 2}, {1, 2, 0}, {2, 0, 1}, {2, 1, 0}};
      auto pm = perms[irand(0, 5)];
      H h3{sh3, x.h.v};
      H hp = permute(h3, pm);
      std::vector<size_t> ps = hp.shape;
      for (auto &e : ps) if (irand(0, 2) == 0) e = 1;
      Val pv = fresh(ps, -1, 1);
      H hq = bcast(hp, pv.h, [](double u, double w) { return u * w + 0.5; });
      Arr t = x.a.view({a, b, C}).permute(pm) * pv.a + 0.5f;
      if (irand(0, 1)) {  // reduce one axis then view to 2-D
        size_t ax = irand(0, 2);
        H hs = sum_any(hq, ax);
        Arr r = t.sum(ax);
        pool.push_back({r.view({hs.shape[0], hs.shape[1]}), H{{hs.shape[0], hs.shape[1]}, hs.v}, "p3sum"});
      } else {
        pool.push_back({t.view({hq.shape[0] * hq.shape[1], hq.shape[2]}), H{{hq.shape[0] * hq.shape[1], hq.shape[2]}, hq.v}, "p3view"});
      }
      return true;
    }
    case 25: {  // batched_dot on a 3-D view, back to 2-D
      if (nd != 2 || x.h.shape[0] < 2) return false;
      size_t R = x.h.shape[0], C = x.h.shape[1], a = divisor(R), b = R / a, N = irand(1, 100);
      Val w = fresh({a, C, N}, -1.0 / std::sqrt(C), 1.0 / std::sqrt(C));
      H h{{R, N}, std::vector<double>(R * N, 0.0)};
      for (size_t g = 0; g < a; g++)
        for (size_t i = 0; i < b; i++)
          for (size_t k = 0; k < C; k++)
            for (size_t n = 0; n < N; n++) h.v[(g * b + i) * N + n] += x.h.v[(g * b + i) * C + k] * w.h.v[(g * C + k) * N + n];
      pool.push_back({x.a.view({a, b, C}).batched_dot(w.a).view({R, N}), h, "bdot"});
      return true;
    }
    case 26: {  // select on a 3-D view
      if (nd != 2 || x.h.shape[0] < 2) return false;
      size_t R = x.h.shape[0], C = x.h.shape[1], a = divisor(R), b = R / a;
      H h3{{a, b, C}, x.h.v};
      size_t ax = irand(0, 2), idx = irand(0, h3.shape[ax] - 1);
      H hs = select(h3, ax, idx);
      if (hs.shape.size() != 2) return false;
      pool.push_back({x.a.view({a, b, C}).select(ax, idx) * 2.0f, unary(hs, [](double v) { return v * 2.0; }), "sel"});
      return true;
    }
    case 27:
    case 28: {  // an N-D chain of views (view, permute, select, slice, transpose,
                // broadcast) over x, then an elementwise node, back to 2-D
      if (nd != 2) return false;
      const size_t n = x.h.v.size();
      std::vector<size_t> sh;
      for (size_t rem = n, k = irand(2, 5); k > 1; k--) {
        size_t d = divisor(rem);
        sh.push_back(d);
        rem /= d;
        if (k == 2) sh.push_back(rem);
      }
      H h{sh, x.h.v};
      Arr a = x.a.view(shape_type(sh.begin(), sh.end()));
      std::string desc = "views" + shp(h);
      for (size_t step_i = 0, steps = irand(1, 4); step_i < steps; step_i++) {
        const size_t d = h.shape.size();
        switch (irand(0, 5)) {
          case 0: {  // permute
            std::vector<size_t> ax(d);
            for (size_t i = 0; i < d; i++) ax[i] = i;
            std::shuffle(ax.begin(), ax.end(), rng_);
            h = permute(h, ax);
            a = a.permute(ax);
            desc += ".p";
            break;
          }
          case 1: {  // select
            if (d < 3) break;
            size_t axis = irand(0, d - 1), idx = irand(0, h.shape[axis] - 1);
            h = select(h, axis, idx);
            a = a.select(axis, idx);
            desc += ".s";
            break;
          }
          case 2: {  // slice along axis 0
            size_t st = irand(0, h.shape[0] - 1), cnt = irand(1, h.shape[0] - st);
            size_t inner = count(std::vector<size_t>(h.shape.begin() + 1, h.shape.end()));
            H o{h.shape, std::vector<double>(h.v.begin() + st * inner, h.v.begin() + (st + cnt) * inner)};
            o.shape[0] = cnt;
            h = o;
            a = a.slice(st, cnt);
            desc += ".sl";
            break;
          }
          case 3: {  // transpose: 2-D or 3-D (the reference reverses the axes of a 3-D array)
            if (d == 3) {
              h = permute(h, {2, 1, 0});
            } else if (d == 2) {
              h = transpose(h);
            } else {
              break;
            }
            a = a.transpose();
            desc += ".t";
            break;
          }
          case 4: {  // reshape to another factorisation of the same count
            const size_t m = h.v.size();
            std::vector<size_t> ns;
            for (size_t rem = m, k = irand(2, 4); k > 1; k--) {
              size_t dd = divisor(rem);
              ns.push_back(dd);
              rem /= dd;
              if (k == 2) ns.push_back(rem);
            }
            h.shape = ns;
            a = a.view(shape_type(ns.begin(), ns.end()));
            desc += ".v";
            break;
          }
          default: {  // broadcast over a new leading axis of 1-3
            if (d >= 5) break;
            size_t k = irand(1, 3);
            std::vector<size_t> ts{k};
            ts.insert(ts.end(), h.shape.begin(), h.shape.end());
            H o{ts, {}};
            for (size_t r = 0; r < k; r++) o.v.insert(o.v.end(), h.v.begin(), h.v.end());
            h = o;
            a = a.broadcast(shape_type(ts.begin(), ts.end()));
            desc += ".b";
            break;
          }
        }
        if (h.v.size() > 2000000) return false;
      }
      if (h.shape.size() < 2) return false;
      H e = unary(h, [](double v) { return v * 1.5 + 0.25; });
      size_t cols = e.shape.back(), rows = e.v.size() / cols;
      Arr r = (a * 1.5f + 0.25f).view({rows, cols});
      pool.push_back({r, H{{rows, cols}, e.v}, desc});
      return true;
    }
    case 29: {  // host writes into an evaluated copy, directly and through a row view
      if (nd != 2) return false;
      const size_t C = x.h.shape[1], n = x.h.v.size();
      Arr y = x.a * 1.0f;
      y.eval();
      H h = x.h;
      for (size_t k = 0, writes = irand(1, 6); k < writes; k++) {
        const size_t i = irand(0, n - 1);
        const float v = float(unif(-2, 2));
        if (irand(0, 1)) {
          y.at(i) = v;
        } else {
          auto row = y.slice(i / C, 1);
          row.at(i % C) = v;
        }
        h.v[i] = v;
      }
      pool.push_back({y, h, "hostw"});
      return true;
    }
    default: {  // residual-style: x + f(x) with x reused
      if (x.h.cols() > 2048) return false;
      Val w = fresh({x.h.cols(), x.h.cols()}, -1.0 / std::sqrt(x.h.cols()), 1.0 / std::sqrt(x.h.cols()));
      if (nd != 2) return false;
      H h = bcast(x.h, dot(x.h, w.h), [](double p, double q) { return p + q; });
      pool.push_back({x.a + x.a.dot(w.a), h, "resid"});
      return true;
    }
  }
}

static bool check(const Val &v, std::string &why) {
  auto &a = v.a;
  size_t n = a.element_count();
  if (n != v.h.v.size()) {
    why = "size " + std::to_string(n) + " vs " + std::to_string(v.h.v.size());
    return false;
  }
  double ss = 0;
  for (double e : v.h.v) ss += e * e;
  double rms = std::sqrt(ss / std::max<size_t>(n, 1));
  for (size_t i = 0; i < n; i++) {
    double got = a.at(i), ref = v.h.v[i];
    if (!(std::fabs(got - ref) <= 1e-3 * rms + 1e-3 * std::fabs(ref) + 1e-6)) {
      char buf[256];
      snprintf(buf, sizeof buf, "element %zu: %.9g vs %.9g (rms %.3g)", i, got, ref, rms);
      why = buf;
      return false;
    }
  }
  return true;
}

int main(int argc, char **argv) {
  uint64_t seed = argc > 1 ? std::stoull(argv[1]) : 1;
  const size_t n_graphs = argc > 2 ? std::stoul(argv[2]) : 200;
  rng_.seed(seed);
  use_gpu();
  size_t graphs = 0, fails = 0;
  while (graphs < n_graphs) {
    std::vector<Val> pool;
    size_t R = irand(1, 4) == 1 ? irand(1, 1100) : irand(1, 300), C = irand(1, 4) == 1 ? irand(1, 1100) : irand(1, 300);
    pool.push_back(fresh({R, C}, -1, 1));
    if (irand(0, 2) == 0) pool.push_back(fresh({C}, -1, 1));
    size_t ops = irand(3, 14), done = 0, tries = 0;
    while (done < ops && tries++ < 200) {
      try {
        size_t before = pool.size();
        if (step(pool)) done++;
        if (pool.size() > before) {
          const auto &ls = pool.back().a.shape();
          if (std::vector<size_t>(ls.begin(), ls.end()) != pool.back().h.shape) {
            printf("FAIL shape, graph %zu: %s library rank %zu shadow %s\n", graphs,
                   pool.back().desc.substr(0, 100).c_str(), ls.size(), shp(pool.back().h).c_str());
            fflush(stdout);
            g_fails++;
            pool.pop_back();
          }
        }
      } catch (const std::exception &e) {
        printf("graph %zu: op threw while building: %s\n", graphs, e.what());
        fflush(stdout);
        fails++;
        break;
      }
      if (pool.back().h.v.size() > 3000000) pool.pop_back();
    }
    std::vector<size_t> roots;
    for (int k = 0; k < 4; k++) roots.push_back(irand(pool.size() > 6 ? pool.size() - 6 : 0, pool.size() - 1));
    try {
      eval(pool[roots[0]].a, pool[roots[1]].a, pool[roots[2]].a, pool[roots[3]].a);
      for (size_t r : roots) {
        std::string why;
        if (!check(pool[r], why)) {
          printf("FAIL graph %zu seed %llu root %zu (%s) shape %s: %s\n", graphs,
                 (unsigned long long)seed, r, pool[r].desc.substr(0, 300).c_str(), shp(pool[r].h).c_str(),
                 why.c_str());
          fflush(stdout);
          fails++;
          break;
        }
      }
    } catch (const std::exception &e) {
      printf("FAIL graph %zu: eval threw: %s\n", graphs, e.what());
      fflush(stdout);
      fails++;
    }
    graphs++;
  }
  fails += g_fails;
  printf("%zu graphs, %zu failures\n", graphs, fails);
  return fails ? 1 : 0;
}
