#pragma once
// sil::array — the reference's C++23 numerical-array front end
// (include/array.h) over the MI355X backend.  The public API follows the
// reference: constructors, views, lazy float arithmetic, dot/linear/
// linear_sigmoid/softmax/layer_norm/sum/min/max/argmax, and sil::eval().
// The implementation is this build's own:
//   * float arrays build a lazy graph (detail::node); evaluation lowers it
//     (detail::evaluate): maximal single-consumer elementwise subgraphs become
//     one fused program launch (one HBM pass for a chain of scalar ops, with
//     the reference's own per-node rounding), everything else one library
//     call per node;
//   * storage is device-resident HBM with a host mirror made current only
//     when the host reads or writes elements (storage.h);
//   * int and bool arrays are handled as in the reference: int elementwise
//     arithmetic on the GPU, the rest on the host.

#include <algorithm>
#include <array>
#include <cmath>
#include <concepts>
#include <cstring>
#include <functional>
#include <initializer_list>
#include <iostream>
#include <iterator>
#include <limits>
#include <memory>
#include <optional>
#include <numeric>
#include <random>
#include <ranges>
#include <span>
#include <sstream>
#include <stdexcept>
#include <string>
#include <tuple>
#include <unordered_map>
#include <unordered_set>
#include <utility>
#include <vector>

#include "gpu.h"

namespace sil {

template <typename T>
concept arithmetic = std::is_arithmetic_v<T>;

using shape_type = std::vector<size_t>;
using strides_type = shape_type;

// Row-major contiguous strides (a scalar has the single stride {1}).
inline strides_type contiguous_strides(const shape_type &shape) {
  if (shape.empty()) return {1};
  strides_type st(shape.size());
  st.back() = 1;
  for (size_t i = shape.size() - 1; i-- > 0;) st[i] = st[i + 1] * shape[i + 1];
  return st;
}

// numpy-style broadcast of two shapes, aligned at the trailing axis
// (include/array.h:38-59).
inline shape_type broadcast_shape(const shape_type &ls, const shape_type &rs) {
  if (ls == rs) return ls;
  if (ls.empty()) return rs;
  if (rs.empty()) return ls;
  const size_t n = std::max(ls.size(), rs.size());
  shape_type out(n);
  for (size_t i = 0; i < n; i++) {
    const size_t a = i + ls.size() >= n ? ls[i + ls.size() - n] : 1;
    const size_t b = i + rs.size() >= n ? rs[i + rs.size() - n] : 1;
    if (a != b && a != 1 && b != 1) throw std::runtime_error("array: invalid operation.");
    out[i] = std::max(a, b);
  }
  return out;
}

inline size_t shape_count(const shape_type &s) {
  size_t n = 1;
  for (auto d : s) n *= d;
  return n;
}

//------------------------------------------------------------------------------
// Lazy graph
//------------------------------------------------------------------------------

namespace detail {

enum class op : uint8_t {
  leaf,
  add, sub, mul, div, pow,           // binary elementwise
  sigmoid, relu, copy,               // unary elementwise (copy: identity)
  sigmoid_backward,                  // elementwise (x, dout)
  softmax, layer_norm,               // row ops
  dot, batched_dot, linear, linear_sigmoid, conv2d,
  sum_axis,
  view,                              // zero-copy strided view of inputs[0]
};

inline bool is_elementwise(op o) { return o >= op::add && o <= op::sigmoid_backward; }
inline bool is_binary(op o) { return o >= op::add && o <= op::pow; }

struct node {
  op operation = op::leaf;
  std::array<std::shared_ptr<node>, 3> inputs{};
  uint8_t num_inputs = 0;

  storage data;  // valid once evaluated
  shape_type shape;
  strides_type strides;
  bool evaluated = false;

  float eps = 0.0f;   // layer_norm
  size_t ksize = 0;   // conv2d kernel size
  size_t axis = 0;    // sum_axis
  size_t view_off = 0;  // view: element offset into inputs[0]'s contiguous result
  int epilogue = 0;     // linear: epilogue fused by the lowering (relu)
  // Folded into a product's epilogue by the lowering: a scalar affine node
  // of the graph (v = fmaf(v, scale, scale_offset), rounded as that node
  // rounds) and a residual add (v + residual, after bias and activation).
  bool use_scale = false;
  float scale = 1.0f, scale_offset = 0.0f;
  std::shared_ptr<node> residual;
  // batched_dot: strides of the output layout when the lowering has the
  // product write straight into a consumer's reordered layout (empty: the
  // contiguous layout of `shape`).
  strides_type out_strides;

  static std::shared_ptr<node> leaf(const storage &s, const shape_type &sh, const strides_type &st) {
    auto n = std::make_shared<node>();
    n->data = s;
    n->shape = sh;
    n->strides = st;
    n->evaluated = true;
    return n;
  }

  static std::shared_ptr<node> make(op o, std::initializer_list<std::shared_ptr<node>> ins,
                                    const shape_type &sh) {
    auto n = std::make_shared<node>();
    n->operation = o;
    for (auto &i : ins) n->inputs[n->num_inputs++] = i;
    n->shape = sh;
    n->strides = contiguous_strides(sh);
    return n;
  }
};

inline void evaluate(const std::vector<node *> &roots);

}  // namespace detail

using lazy_node = detail::node;

//------------------------------------------------------------------------------
// Nested initializer lists (array{{1,2},{3,4}})
//------------------------------------------------------------------------------

template <value_type T, size_t I>
struct nested_initializer_list_ {
  using type = std::initializer_list<typename nested_initializer_list_<T, I - 1>::type>;
};
template <value_type T>
struct nested_initializer_list_<T, 0> {
  using type = T;
};
template <value_type T, size_t I>
using nested_initializer_list = typename nested_initializer_list_<T, I>::type;

namespace detail {

template <typename L>
void nested_shape(const L &l, shape_type &s, size_t depth) {
  if constexpr (requires { l.begin(); l.size(); }) {
    if (s.size() <= depth) s.push_back(l.size());
    if (l.size() > 0) nested_shape(*l.begin(), s, depth + 1);
  }
}

template <typename L>
size_t nested_count(const L &l) {
  if constexpr (requires { l.begin(); l.size(); }) {
    size_t n = 0;
    for (const auto &x : l) n += nested_count(x);
    return n;
  } else {
    return 1;
  }
}

template <typename T, typename L>
void nested_copy(T *&dst, const L &l) {
  if constexpr (requires { l.begin(); l.size(); }) {
    for (const auto &x : l) nested_copy(dst, x);
  } else {
    *dst++ = static_cast<T>(l);
  }
}

}  // namespace detail

//------------------------------------------------------------------------------

template <value_type T>
class array;

template <value_type T, bool IsConst>
class element_iterator_;
template <value_type T, bool IsConst>
class row_iterator_;

template <value_type T>
class array {
  template <value_type U>
  friend class array;

 public:
  using value_t = T;

  array() = default;
  array(const array &) = default;
  array(array &&) = default;
  array &operator=(const array &) = default;
  array &operator=(array &&) = default;

  array(const shape_type &shape, T val) {
    reshape_raw_(shape);
    allocate_();
    constants(val);
  }
  template <std::input_iterator It>
  array(const shape_type &shape, It it) {
    reshape_raw_(shape);
    allocate_();
    set(it);
  }
  template <std::ranges::input_range R>
    requires(!std::is_same_v<std::remove_cvref_t<R>, array>)
  array(const shape_type &shape, R &&r) {
    reshape_raw_(shape);
    allocate_();
    set(std::ranges::begin(r));
  }
  template <std::ranges::input_range R>
    requires(!std::is_same_v<std::remove_cvref_t<R>, array> &&
             !std::is_same_v<std::remove_cvref_t<R>, shape_type>)
  explicit array(R &&r) {
    std::vector<T> tmp;
    for (auto &&x : r) tmp.push_back(static_cast<T>(x));
    reshape_raw_({tmp.size()});
    allocate_();
    set(tmp.begin());
  }
  array(T val) : array(shape_type{}, val) {}

  array(nested_initializer_list<T, 1> l) { init_list_(l); }
  array(nested_initializer_list<T, 2> l) { init_list_(l); }
  array(nested_initializer_list<T, 3> l) { init_list_(l); }
  array(nested_initializer_list<T, 4> l) { init_list_(l); }

  //----------------------------------------------------------------------------

  template <value_type U = T>
  array<U> clone() const {
    array<U> tmp(shape_, U{});
    for (size_t i = 0; i < element_count(); i++) tmp.at(i) = static_cast<U>(at(i));
    return tmp;
  }

  void eval() const { ensure_evaluated_(); }
  std::shared_ptr<lazy_node> lazy_node_ptr() const { return node_; }

  //----------------------------------------------------------------------------

  array<bool> operator==(const array &rhs) const { return compare_(rhs, std::equal_to<>{}); }
  array<bool> operator!=(const array &rhs) const { return compare_(rhs, std::not_equal_to<>{}); }
  array<bool> operator>(const array &rhs) const { return compare_(rhs, std::greater<>{}); }
  array<bool> operator<(const array &rhs) const { return compare_(rhs, std::less<>{}); }
  array<bool> operator>=(const array &rhs) const { return compare_(rhs, std::greater_equal<>{}); }
  array<bool> operator<=(const array &rhs) const { return compare_(rhs, std::less_equal<>{}); }

  //----------------------------------------------------------------------------

  size_t buffer_element_count() const {
    ensure_evaluated_();
    return storage_.len;
  }
  size_t buffer_bytes() const { return buffer_element_count() * sizeof(T); }

  // Host pointer to the first element of this array's window; waits for the
  // GPU when the data is still being computed (include/array.h:951-958).
  T *buffer_data() {
    ensure_evaluated_();
    return storage_.template host_out<T>();
  }
  const T *buffer_data() const {
    ensure_evaluated_();
    return storage_.template host_in<T>();
  }
  std::span<T> buffer_span() { return std::span<T>(buffer_data(), buffer_element_count()); }
  std::span<const T> buffer_span() const {
    return std::span<const T>(buffer_data(), buffer_element_count());
  }

  //----------------------------------------------------------------------------

  size_t element_count() const { return shape_count(shape_); }
  size_t length() const {
    if (shape_.empty()) throw std::runtime_error("array: cannot call with a scalar value.");
    return shape_[0];
  }
  size_t dimension() const { return shape_.size(); }
  const shape_type &shape() const { return shape_; }
  const strides_type &strides() const { return strides_; }

  void reshape(const shape_type &shape) {
    ensure_evaluated_();
    if (storage_ && shape_count(shape) != element_count() && storage_.len < shape_count(shape))
      throw std::runtime_error("array: invalid shape for reshape.");
    if (storage_ && !is_contiguous_()) *this = materialize_();
    reshape_raw_(shape);
  }

  // Zero-copy broadcast view to `target_shape` (include/array.h:1008-1049).
  array broadcast(const shape_type &target_shape) const {
    ensure_evaluated_();
    if (target_shape.size() < dimension())
      throw std::runtime_error("array: invalid shape for broadcast.");
    const size_t diff = target_shape.size() - dimension();
    for (size_t i = 0; i < dimension(); i++)
      if (shape_[i] != target_shape[i + diff] && shape_[i] != 1)
        throw std::runtime_error("array: invalid shape for broadcast.");
    if (target_shape == shape_) return *this;
    array tmp = *this;
    tmp.node_.reset();
    tmp.shape_ = target_shape;
    tmp.strides_.assign(target_shape.size(), 0);
    for (size_t i = diff; i < target_shape.size(); i++) {
      const size_t s = i - diff;
      tmp.strides_[i] = (shape_[s] == 1 && target_shape[i] != 1) ? 0 : strides_[s];
    }
    return tmp;
  }

  // 1-D -> {1, n}; {1, n} -> {n}; 2-D: zero-copy stride swap; 3-D: reversed
  // axes, copied (include/array.h:1051-1099).
  array transpose() const {
    // A lazy matrix stays in the graph as a transposed view; products read
    // it in place (transposed operand), elementwise programs by strides.
    if (node_ && !node_->evaluated && dimension() == 2 && shape_[0] != 1)
      return permute({1, 0});
    ensure_evaluated_();
    if (dimension() == 1) {
      array tmp = *this;
      tmp.node_.reset();
      tmp.shape_ = {1, element_count()};
      tmp.strides_ = {element_count(), 1};
      if (!is_contiguous_()) return materialize_().transpose();
      return tmp;
    }
    if (dimension() == 2) {
      // {1, n} -> {n} for every row view, as the reference does; the vector
      // keeps the row's element stride (a row of a transposed view is not
      // contiguous; the reference's unit stride would read other elements).
      if (shape_[0] == 1) {
        array tmp = *this;
        tmp.node_.reset();
        tmp.shape_ = {shape_[1]};
        tmp.strides_ = {strides_[1]};
        return tmp;
      }
      array tmp = *this;
      tmp.node_.reset();
      tmp.shape_ = {shape_[1], shape_[0]};
      tmp.strides_ = {strides_[1], strides_[0]};
      return tmp;
    }
    if (dimension() == 3) {
      auto shape = shape_;
      std::ranges::reverse(shape);
      auto tmp = make_uninit_(shape);
      T *out = tmp.storage_.template host_out<T>();
      const auto st = contiguous_strides(shape);
      for (size_t z = 0; z < shape_[0]; z++)
        for (size_t y = 0; y < shape_[1]; y++)
          for (size_t x = 0; x < shape_[2]; x++)
            out[x * st[0] + y * st[1] + z * st[2]] = (*this)[z, y, x];
      return tmp;
    }
    throw std::runtime_error("array: can't do `transpose` operation.");
  }

  //----------------------------------------------------------------------------

  T &at() { return *buffer_data(); }
  const T &at() const { return *buffer_data(); }
  T &at(size_t i) {
    bounds_check_(i);
    return buffer_data()[index_of_(i)];
  }
  const T &at(size_t i) const {
    bounds_check_(i);
    return buffer_data()[index_of_(i)];
  }
  T &operator[](size_t x, size_t y) {
    bounds_check_(x, y);
    return buffer_data()[strides_[0] * x + strides_[1] * y];
  }
  const T &operator[](size_t x, size_t y) const {
    bounds_check_(x, y);
    return buffer_data()[strides_[0] * x + strides_[1] * y];
  }
  T &operator[](size_t x, size_t y, size_t z) {
    bounds_check_(x, y, z);
    return buffer_data()[strides_[0] * x + strides_[1] * y + strides_[2] * z];
  }
  const T &operator[](size_t x, size_t y, size_t z) const {
    bounds_check_(x, y, z);
    return buffer_data()[strides_[0] * x + strides_[1] * y + strides_[2] * z];
  }
  T &at(const std::vector<size_t> &position) { return buffer_data()[offset_of_(position)]; }
  const T &at(const std::vector<size_t> &position) const {
    return buffer_data()[offset_of_(position)];
  }

  template <size_t I>
  auto take() const {
    if constexpr (I == 0) return std::tuple<>();
    else return std::tuple_cat(take<I - 1>(), std::tuple<T>(at(I - 1)));
  }

  //----------------------------------------------------------------------------

  // Zero-copy view of row `row` (include/array.h:1157-1175).
  array operator[](size_t row) const {
    if (dimension() == 0 || row >= shape_[0])
      throw std::runtime_error("array: row is out of bounds.");
    ensure_evaluated_();
    array tmp(*this);
    tmp.node_.reset();
    tmp.shape_.erase(tmp.shape_.begin());
    tmp.strides_.erase(tmp.strides_.begin());
    if (tmp.shape_.empty()) tmp.strides_ = {1};
    tmp.storage_.off = storage_.off + strides_[0] * row;
    tmp.storage_.len = tmp.shape_.empty() ? 1 : strides_[0];
    return tmp;
  }

  // Zero-copy view of rows [start, start + count) (include/array.h:1177-1187).
  array slice(size_t start, size_t count) const {
    ensure_evaluated_();
    if (dimension() == 0 || start + count > shape_[0])
      throw std::runtime_error("array: slice is out of bounds.");
    array tmp(*this);
    tmp.node_.reset();
    tmp.shape_[0] = count;
    tmp.storage_.off = storage_.off + strides_[0] * start;
    tmp.storage_.len = count * strides_[0];
    return tmp;
  }

  //----------------------------------------------------------------------------

  auto element_begin() { return element_iterator_<T, false>(this, 0); }
  auto element_end() { return element_iterator_<T, false>(this, element_count()); }
  auto element_cbegin() const { return element_iterator_<T, true>(this, 0); }
  auto element_cend() const { return element_iterator_<T, true>(this, element_count()); }

  auto elements() { return std::ranges::subrange(element_begin(), element_end()); }
  auto elements() const { return std::ranges::subrange(element_cbegin(), element_cend()); }

  auto begin() { return row_iterator_<T, false>(this, 0); }
  auto end() { return row_iterator_<T, false>(this, shape_.empty() ? 0 : shape_[0]); }
  auto begin() const { return row_iterator_<T, true>(this, 0); }
  auto end() const { return row_iterator_<T, true>(this, shape_.empty() ? 0 : shape_[0]); }
  auto cbegin() const { return begin(); }
  auto cend() const { return end(); }

  // rows(): the rows as arrays; rows<N>(): the rows' first N elements as
  // tuples (include/array.h:706-755).
  template <size_t N = 0>
  auto rows() {
    if constexpr (N == 0) {
      return std::ranges::subrange(begin(), end());
    } else {
      std::vector<decltype(std::declval<array>().template take<N>())> out;
      for (size_t r = 0; r < length(); r++) out.push_back((*this)[r].template take<N>());
      return out;
    }
  }
  template <size_t N = 0>
  auto rows() const {
    if constexpr (N == 0) {
      return std::ranges::subrange(begin(), end());
    } else {
      std::vector<decltype(std::declval<const array>().template take<N>())> out;
      for (size_t r = 0; r < length(); r++) out.push_back((*this)[r].template take<N>());
      return out;
    }
  }

  //----------------------------------------------------------------------------

  template <std::input_iterator It>
  void set(It it) {
    ensure_evaluated_();
    T *p = storage_.template host_out<T>();
    for (size_t i = 0; i < element_count(); i++) p[index_of_(i)] = static_cast<T>(*it++);
    node_.reset();
  }
  void set(std::initializer_list<T> l) { set(l.begin()); }

  // Fill: on the device for a large contiguous float/int array (no host
  // mirror is created), otherwise on the host, so small arrays and scalars
  // stay host-readable (scalar operands fold into fused programs on the
  // host, see detail::program_builder).
  void constants(T val) {
    ensure_evaluated_();
    if constexpr (sizeof(T) == 4) {
      if (device_ == Device::GPU && element_count() >= 4096 && is_contiguous_() &&
          element_count() == storage_.len) {
        uint32_t bits;
        std::memcpy(&bits, &val, 4);
        gpu::launched_(silgpu_fill_u32(storage_.template dev_out<T>(), bits,
                                       int64_t(storage_.len)),
                       "fill");
        node_.reset();
        return;
      }
    }
    T *p = storage_.template host_out<T>();
    for (size_t i = 0; i < element_count(); i++) p[index_of_(i)] = val;
    node_.reset();
  }
  void zeros() { constants(T(0)); }
  void ones() { constants(T(1)); }
  // Uniform [0, 1) from a per-thread Mersenne twister, as the reference
  // (include/array.h:1284-1290).
  void random() {
    thread_local std::mt19937 gen(std::random_device{}());
    std::uniform_real_distribution<float> dist(0.0f, 1.0f);
    ensure_evaluated_();
    T *p = storage_.template host_out<T>();
    for (size_t i = 0; i < element_count(); i++) p[index_of_(i)] = static_cast<T>(dist(gen));
    node_.reset();
  }

  //----------------------------------------------------------------------------

  array operator+(const array &rhs) const { return binary_(detail::op::add, rhs); }
  array operator-(const array &rhs) const { return binary_(detail::op::sub, rhs); }
  array operator*(const array &rhs) const { return binary_(detail::op::mul, rhs); }
  array operator/(const array &rhs) const { return binary_(detail::op::div, rhs); }
  array pow(const array &rhs) const { return binary_(detail::op::pow, rhs); }

  // Compound assignment: out of place for float (the result is a new lazy
  // node, as the reference's GPU mode, include/array.h:2614-2628).
  void operator+=(const array &rhs) { *this = *this + rhs; }
  void operator-=(const array &rhs) { *this = *this - rhs; }
  void operator*=(const array &rhs) { *this = *this * rhs; }
  void operator/=(const array &rhs) { *this = *this / rhs; }

  //----------------------------------------------------------------------------

  array dot(const array &rhs) const;
  // Batched product over the leading axes: {..., M, K} x {..., K, N} ->
  // {..., M, N} (the reference's {B, M, K} x {B, K, N}, include/array.h:1360-1373,
  // extended to strided and higher-rank operands).
  array batched_dot(const array &rhs) const;

  // Zero-copy views (no reference counterpart; the reference copies on 3-D
  // transpose, include/array.h:1079-1096).  Lazy when the array is lazy.
  //   view(shape)        the same elements under a new contiguous shape
  //   permute(axes)      axes reordered: result axis i is source axis axes[i]
  //   select(axis, i)    index i of one axis; that axis is removed
  array view(const shape_type &shape) const;
  array permute(const std::vector<size_t> &axes) const;
  array select(size_t axis, size_t index) const;
  array linear(const array &W, const array &b) const;

  array<float> sigmoid() const;
  array<float> sigmoid_backward(const array<float> &dout) const;
  array<float> linear_sigmoid(const array &W, const array &b) const;
  array<float> relu() const;
  array<float> layer_norm(const array<float> &gamma, const array<float> &beta,
                          float eps = 1e-5f) const;
  // NHWC input [N, H, W, C_in] with an OHWI weight [C_out, K, K, C_in]:
  // [N, H, W, C_out], stride 1, zero padding K / 2 (include/array.h:1508-1517).
  array<float> conv2d(const array<float> &weight, size_t kernel_size) const;

  //----------------------------------------------------------------------------

  T sum() const;
  array sum(size_t axis) const;
  float mean() const { return static_cast<float>(sum()) / static_cast<float>(element_count()); }
  array<float> mean(size_t axis) const;
  T min() const;
  T max() const;

  size_t count() const {
    size_t n = 0;
    for (size_t i = 0; i < element_count(); i++) n += !!at(i);
    return n;
  }
  bool all(arithmetic auto val) const {
    for (size_t i = 0; i < element_count(); i++)
      if (!(at(i) == static_cast<T>(val))) return false;
    return true;
  }
  template <typename F>
    requires std::invocable<F, T>
  bool all(F fn) const {
    for (size_t i = 0; i < element_count(); i++)
      if (!fn(at(i))) return false;
    return true;
  }

  array<float> softmax() const;
  array<int> argmax() const;
  float mean_square_error(const array &rhs) const {
    return (*this - rhs).pow(array(static_cast<T>(2))).mean();
  }
  template <value_type U = T>
  array<U> one_hot(size_t class_count) const {
    if (dimension() != 1)
      throw std::runtime_error("array: one_hot is available only for 1 dimension array.");
    array<U> tmp({shape_[0], class_count}, U{});
    for (size_t i = 0; i < element_count(); i++)
      tmp[i, static_cast<size_t>(at(i))] = U(1);
    return tmp;
  }

  //----------------------------------------------------------------------------

  std::string print_shape_type(const shape_type &shape) const {
    std::string s = "{";
    for (size_t i = 0; i < shape.size(); i++) {
      if (i) s += ", ";
      s += std::to_string(shape[i]);
    }
    return s + "}";
  }
  std::string print_shape() const { return print_shape_type(shape_); }
  std::string print_strides() const { return print_shape_type(strides_); }
  std::string print_data_type() const {
    if constexpr (std::is_same_v<T, float>) return "float";
    else if constexpr (std::is_same_v<T, int>) return "int";
    else return "bool";
  }
  std::string print_info() const {
    std::ostringstream os;
    os << "dtype: " << print_data_type() << ", dim: " << dimension()
       << ", shape: " << print_shape() << ", strides: " << print_strides();
    return os.str();
  }
  std::string print_array() const {
    std::ostringstream os;
    if (dimension() == 0) {
      print_value_(os, at());
      return os.str();
    }
    size_t idx = 0;
    print_level_(os, 0, idx);
    return os.str();
  }

  //----------------------------------------------------------------------------
  // Backend access (also used by the reference's boundary-level tests).

  const storage &storage_ref() const {
    ensure_evaluated_();
    return storage_;
  }

  // An evaluated array over existing storage (no copy).
  static array view_(const storage &s, const shape_type &shape, const strides_type &strides) {
    array a;
    a.storage_ = s;
    a.shape_ = shape;
    a.strides_ = strides;
    return a;
  }

  static array make_uninit_(const shape_type &shape) {
    array a;
    a.reshape_raw_(shape);
    a.allocate_();
    return a;
  }

  bool is_contiguous_() const {
    if (shape_.empty()) return true;
    return strides_ == contiguous_strides(shape_);
  }

  // A contiguous copy of this (possibly strided or broadcast) view.
  array materialize_() const;

 private:
  shape_type shape_;
  strides_type strides_;
  storage storage_;
  std::shared_ptr<detail::node> node_;

  void reshape_raw_(const shape_type &shape) {
    shape_ = shape;
    strides_ = contiguous_strides(shape);
  }

  void allocate_() {
    const size_t len = element_count();
    storage_ = storage::make_device(len * sizeof(T));
    storage_.off = 0;
    storage_.len = len;
  }

  template <typename L>
  void init_list_(const L &l) {
    shape_type s;
    detail::nested_shape(l, s, 0);
    reshape_raw_(s);
    allocate_();
    if (detail::nested_count(l) != element_count())
      throw std::runtime_error("array: invalid initializer list.");
    T *p = storage_.template host_out<T>();
    detail::nested_copy(p, l);
  }

  void ensure_evaluated_() const {
    if (!node_) return;
    if (!node_->evaluated) detail::evaluate({node_.get()});
    if (!storage_ || storage_.buf != node_->data.buf || storage_.off != node_->data.off) {
      auto &self = const_cast<array &>(*this);
      self.shape_ = node_->shape;
      self.strides_ = node_->strides;
      self.storage_ = node_->data;
    }
  }

  // Buffer offset (relative to storage_.off) of the i-th element in
  // row-major order of this view.
  size_t index_of_(size_t i) const {
    if (is_contiguous_()) return i;
    size_t off = 0;
    for (size_t d = shape_.size(); d-- > 0;) {
      off += (i % shape_[d]) * strides_[d];
      i /= shape_[d];
    }
    return off;
  }
  size_t offset_of_(const std::vector<size_t> &pos) const {
    size_t off = 0;
    for (size_t i = 0; i < pos.size(); i++) off += strides_[i] * pos[i];
    return off;
  }

  void bounds_check_(size_t i) const {
    if (strides_.empty() || i >= element_count())
      throw std::runtime_error("array: index is out of bounds.");
  }
  void bounds_check_(size_t x, size_t y) const {
    if (dimension() != 2 || x >= shape_[0] || y >= shape_[1])
      throw std::runtime_error("array: (x, y) is out of bounds.");
  }
  void bounds_check_(size_t x, size_t y, size_t z) const {
    if (dimension() != 3 || x >= shape_[0] || y >= shape_[1] || z >= shape_[2])
      throw std::runtime_error("array: (x, y, z) is out of bounds.");
  }

  static std::shared_ptr<detail::node> to_node_(const array &a) {
    if (a.node_ && !a.node_->evaluated) return a.node_;
    if (a.node_ && a.node_->evaluated && !a.storage_)
      return detail::node::leaf(a.node_->data, a.node_->shape, a.node_->strides);
    return detail::node::leaf(a.storage_, a.shape_, a.strides_);
  }

  static array from_node_(std::shared_ptr<detail::node> n) {
    array a;
    a.shape_ = n->shape;
    a.strides_ = n->strides;
    a.node_ = std::move(n);
    return a;
  }

  static void require_gpu_() {
    if (device_ == Device::CPU)
      throw std::runtime_error(
          "array: float evaluation needs the GPU backend (sil::use_gpu()); the CPU backend "
          "is not part of this build.");
  }

  array binary_(detail::op o, const array &rhs) const;
  array int_binary_(detail::op o, const array &rhs) const;
  array host_binary_(detail::op o, const array &rhs, const shape_type &shape) const;

  template <typename F>
  array<bool> compare_(const array &rhs, F f) const {
    const auto shape = broadcast_shape(shape_, rhs.shape_);
    auto l = broadcast(shape);
    auto r = rhs.broadcast(shape);
    array<bool> out(shape, false);
    bool *o = out.buffer_data();
    for (size_t i = 0; i < out.element_count(); i++) o[i] = f(l.at(i), r.at(i));
    return out;
  }

  static void print_value_(std::ostream &os, const T &v) {
    if constexpr (std::is_same_v<T, bool>) os << (v ? "true" : "false");
    else os << v;
  }
  void print_level_(std::ostream &os, size_t dim, size_t &idx) const {
    os << '{';
    for (size_t i = 0; i < shape_[dim]; i++) {
      if (i) {
        os << ", ";
        if (dim + 1 < dimension()) os << '\n' << std::string(dim + 1, ' ');
      }
      if (dim + 1 == dimension()) print_value_(os, at(idx++));
      else print_level_(os, dim + 1, idx);
    }
    os << '}';
  }
};

//------------------------------------------------------------------------------
// Iterators
//------------------------------------------------------------------------------

template <value_type T, bool IsConst>
class element_iterator_ {
  using arr_ptr = std::conditional_t<IsConst, const array<T> *, array<T> *>;

 public:
  using difference_type = std::ptrdiff_t;
  using value_type = T;
  using reference = std::conditional_t<IsConst, const T &, T &>;
  using iterator_concept = std::forward_iterator_tag;

  element_iterator_() = default;
  element_iterator_(arr_ptr a, size_t i) : a_(a), i_(i) {}
  reference operator*() const { return a_->at(i_); }
  element_iterator_ &operator++() {
    ++i_;
    return *this;
  }
  element_iterator_ operator++(int) {
    auto t = *this;
    ++i_;
    return t;
  }
  bool operator==(const element_iterator_ &o) const { return i_ == o.i_; }

 private:
  arr_ptr a_ = nullptr;
  size_t i_ = 0;
};

template <value_type T, bool IsConst>
class row_iterator_ {
  using arr_ptr = std::conditional_t<IsConst, const array<T> *, array<T> *>;

 public:
  using difference_type = std::ptrdiff_t;
  using value_type = array<T>;
  using iterator_concept = std::forward_iterator_tag;

  row_iterator_() = default;
  row_iterator_(arr_ptr a, size_t i) : a_(a), i_(i) {}
  array<T> operator*() const { return (*a_)[i_]; }
  row_iterator_ &operator++() {
    ++i_;
    return *this;
  }
  row_iterator_ operator++(int) {
    auto t = *this;
    ++i_;
    return t;
  }
  bool operator==(const row_iterator_ &o) const { return i_ == o.i_; }

 private:
  arr_ptr a_ = nullptr;
  size_t i_ = 0;
};

//------------------------------------------------------------------------------
// Lazy float ops
//------------------------------------------------------------------------------

template <value_type T>
inline array<T> array<T>::binary_(detail::op o, const array &rhs) const {
  if constexpr (std::is_same_v<T, float>) {
    auto shape = broadcast_shape(shape_, rhs.shape_);
    return from_node_(detail::node::make(o, {to_node_(*this), to_node_(rhs)}, shape));
  } else {
    return int_binary_(o, rhs);
  }
}

// int arithmetic, eager on the GPU (the reference's msl::add<int> path,
// include/gpu.h:1331-1369); bool arithmetic on the host.
template <value_type T>
inline array<T> array<T>::int_binary_(detail::op o, const array &rhs) const {
  const auto shape = broadcast_shape(shape_, rhs.shape_);
  if constexpr (std::is_same_v<T, int>) {
    if (device_ == Device::CPU) return host_binary_(o, rhs, shape);
    auto full = [&](const array &a) {
      return (a.shape_ == shape && a.is_contiguous_()) ? a : a.broadcast(shape).materialize_();
    };
    auto l = full(*this);
    auto r = full(rhs);
    auto out = make_uninit_(shape);
    int opc = o == detail::op::add ? SILGPU_ADD : o == detail::op::sub ? SILGPU_SUB
              : o == detail::op::mul ? SILGPU_MUL : o == detail::op::div ? SILGPU_DIV
                                                                        : SILGPU_POW;
    const int32_t *lp = l.storage_.template dev_in<int32_t>();
    const int32_t *rp = r.storage_.template dev_in<int32_t>();
    gpu::launched_(silgpu_binary_i32(opc, lp, int64_t(l.storage_.len), rp,
                                     int64_t(r.storage_.len),
                                     out.storage_.template dev_out<int32_t>(),
                                     int64_t(out.element_count())),
                   "arithmetic");
    return out;
  } else {
    return host_binary_(o, rhs, shape);
  }
}

// Host evaluation of int / bool arithmetic (the reference's CPU mode for
// non-float arrays, include/cpu.h:76-237).
template <value_type T>
inline array<T> array<T>::host_binary_(detail::op o, const array &rhs,
                                       const shape_type &shape) const {
  {
    auto l = broadcast(shape);
    auto r = rhs.broadcast(shape);
    array out(shape, T{});
    T *p = out.buffer_data();
    for (size_t i = 0; i < out.element_count(); i++) {
      const int a = l.at(i), b = r.at(i);
      int v = o == detail::op::add ? a + b : o == detail::op::sub ? a - b
              : o == detail::op::mul ? a * b : o == detail::op::div ? (b ? a / b : 0)
              // powi of the reference: round(pow(float(a), float(b)))
              : int(std::rint(std::pow(float(a), float(b))));
      p[i] = static_cast<T>(v);
    }
    return out;
  }
}

template <value_type T>
inline array<T> array<T>::materialize_() const {
  ensure_evaluated_();
  auto out = make_uninit_(shape_);
  if constexpr (std::is_same_v<T, float>) {
    if (element_count() == 0) return out;
    // One-input program: a strided / broadcast gather into contiguous memory.
    if (shape_.size() > SILGPU_PROG_MAX_DIMS) throw std::runtime_error("array: too many axes.");
    silgpu_program p{};
    p.ndim = static_cast<int32_t>(shape_.size());
    for (size_t d = 0; d < shape_.size(); d++) {
      p.shape[d] = int64_t(shape_[d]);
      p.inputs[0].strides[d] = int64_t(strides_[d]);
    }
    p.n_inputs = 1;
    p.inputs[0].ptr = storage_.template dev_in<float>();
    p.n_instrs = 1;
    p.instrs[0] = {SILGPU_PI_LOAD, 0, 0, 0, 0.0f, 0.0f};
    p.out_reg = 0;
    gpu::program(p, out.storage_);
  } else {
    T *o = out.storage_.template host_out<T>();
    for (size_t i = 0; i < element_count(); i++) o[i] = at(i);
  }
  return out;
}

template <value_type T>
inline array<T> array<T>::dot(const array &rhs) const {
  shape_type out_shape;
  if (dimension() == 2 && rhs.dimension() == 2 && shape_[1] == rhs.shape_[0])
    out_shape = {shape_[0], rhs.shape_[1]};
  else if (dimension() == 1 && rhs.dimension() == 2 && shape_[0] == rhs.shape_[0])
    out_shape = {rhs.shape_[1]};
  else if (dimension() == 2 && rhs.dimension() == 1 && shape_[1] == rhs.shape_[0])
    out_shape = {shape_[0]};
  else if (dimension() == 1 && rhs.dimension() == 1 && shape_[0] == rhs.shape_[0])
    out_shape = {};
  else
    throw std::runtime_error("array: can't do `dot` operation.");
  if constexpr (std::is_same_v<T, float>) {
    return from_node_(detail::node::make(detail::op::dot, {to_node_(*this), to_node_(rhs)},
                                         out_shape));
  } else {
    // Integer products on the host, as the reference (include/cpu.h:239-264).
    // A vector operand as a one-row (left) or one-column (right) view.
    auto a = dimension() == 1 ? broadcast({1, shape_[0]}) : *this;
    auto b = rhs;
    if (rhs.dimension() == 1) {
      b.shape_ = {rhs.shape_[0], 1};
      b.strides_ = {rhs.strides_[0], 1};
    }
    const size_t M = a.shape_[0], K = a.shape_[1], N = b.shape_[1];
    array out(out_shape, T{});
    T *o = out.buffer_data();
    for (size_t i = 0; i < M; i++)
      for (size_t j = 0; j < N; j++) {
        T s{};
        for (size_t k = 0; k < K; k++) s += a[i, k] * b[k, j];
        o[i * N + j] = s;
      }
    return out;
  }
}

template <value_type T>
inline array<T> array<T>::batched_dot(const array &rhs) const {
  static_assert(std::is_same_v<T, float>, "batched_dot requires float");
  const size_t nd = dimension();
  if (nd < 3 || rhs.dimension() != nd)
    throw std::runtime_error("batched_dot: requires 3D arrays");
  for (size_t d = 0; d + 2 < nd; d++)
    if (shape_[d] != rhs.shape_[d]) throw std::runtime_error("batched_dot: shape mismatch");
  if (shape_[nd - 1] != rhs.shape_[nd - 2]) throw std::runtime_error("batched_dot: shape mismatch");
  auto out_shape = shape_;
  out_shape[nd - 1] = rhs.shape_[nd - 1];
  return from_node_(detail::node::make(detail::op::batched_dot, {to_node_(*this), to_node_(rhs)},
                                       out_shape));
}

// A view is (shape, strides, offset) over the contiguous result of a source
// that is not itself a view, so views of views compose by arithmetic on
// those three.
template <value_type T>
inline array<T> array<T>::view(const shape_type &shape) const {
  if (shape_count(shape) != element_count())
    throw std::runtime_error("array: invalid shape for view.");
  if (node_ && !node_->evaluated) {
    if (node_->operation == detail::op::view) {
      if (node_->strides != contiguous_strides(node_->shape)) {
        // Gather the strided view into a contiguous result first (a copy
        // node, fused into its producer's or consumer's program).
        auto c = detail::node::make(detail::op::copy, {node_}, node_->shape);
        return from_node_(detail::node::make(detail::op::view, {c}, shape));
      }
      auto n = detail::node::make(detail::op::view, {node_->inputs[0]}, shape);
      n->view_off = node_->view_off;
      return from_node_(std::move(n));
    }
    auto n = detail::node::make(detail::op::view, {node_}, shape);
    return from_node_(std::move(n));
  }
  ensure_evaluated_();
  array src = is_contiguous_() ? *this : materialize_();
  array tmp = src;
  tmp.node_.reset();
  tmp.shape_ = shape;
  tmp.strides_ = contiguous_strides(shape);
  return tmp;
}

template <value_type T>
inline array<T> array<T>::permute(const std::vector<size_t> &axes) const {
  if (axes.size() != dimension()) throw std::runtime_error("array: invalid permutation.");
  std::vector<bool> seen(axes.size(), false);
  for (auto a : axes) {
    if (a >= axes.size() || seen[a]) throw std::runtime_error("array: invalid permutation.");
    seen[a] = true;
  }
  auto apply = [&](const shape_type &sh, const strides_type &st, shape_type &nsh,
                   strides_type &nst) {
    nsh.resize(axes.size());
    nst.resize(axes.size());
    for (size_t i = 0; i < axes.size(); i++) {
      nsh[i] = sh[axes[i]];
      nst[i] = st[axes[i]];
    }
  };
  if (node_ && !node_->evaluated) {
    const bool v = node_->operation == detail::op::view;
    auto n = std::make_shared<detail::node>();
    n->operation = detail::op::view;
    n->inputs[0] = v ? node_->inputs[0] : node_;
    n->num_inputs = 1;
    n->view_off = v ? node_->view_off : 0;
    apply(node_->shape, node_->strides, n->shape, n->strides);
    return from_node_(std::move(n));
  }
  ensure_evaluated_();
  array tmp = *this;
  tmp.node_.reset();
  apply(shape_, strides_, tmp.shape_, tmp.strides_);
  return tmp;
}

template <value_type T>
inline array<T> array<T>::select(size_t axis, size_t index) const {
  if (axis >= dimension() || index >= shape_[axis])
    throw std::runtime_error("array: select is out of bounds.");
  if (node_ && !node_->evaluated) {
    const bool v = node_->operation == detail::op::view;
    auto n = std::make_shared<detail::node>();
    n->operation = detail::op::view;
    n->inputs[0] = v ? node_->inputs[0] : node_;
    n->num_inputs = 1;
    n->view_off = (v ? node_->view_off : 0) + node_->strides[axis] * index;
    n->shape = node_->shape;
    n->strides = node_->strides;
    n->shape.erase(n->shape.begin() + axis);
    n->strides.erase(n->strides.begin() + axis);
    if (n->shape.empty()) n->strides = {1};
    return from_node_(std::move(n));
  }
  ensure_evaluated_();
  array tmp = *this;
  tmp.node_.reset();
  tmp.storage_.off = storage_.off + strides_[axis] * index;
  tmp.shape_.erase(tmp.shape_.begin() + axis);
  tmp.strides_.erase(tmp.strides_.begin() + axis);
  if (tmp.shape_.empty()) tmp.strides_ = {1};
  return tmp;
}

template <value_type T>
inline array<T> array<T>::linear(const array &W, const array &b) const {
  if constexpr (std::is_same_v<T, float>) {
    if (dimension() != 2 || W.dimension() != 2 || shape_[1] != W.shape_[0])
      throw std::runtime_error("array: can't do `linear` operation.");
    return from_node_(detail::node::make(detail::op::linear,
                                         {to_node_(*this), to_node_(W), to_node_(b)},
                                         {shape_[0], W.shape_[1]}));
  } else {
    return dot(W) + b;
  }
}

template <value_type T>
inline array<float> array<T>::sigmoid() const {
  if constexpr (std::is_same_v<T, float>)
    return from_node_(detail::node::make(detail::op::sigmoid, {to_node_(*this)}, shape_));
  else
    return clone<float>().sigmoid();
}

template <value_type T>
inline array<float> array<T>::sigmoid_backward(const array<float> &dout) const {
  if constexpr (std::is_same_v<T, float>)
    return from_node_(detail::node::make(detail::op::sigmoid_backward,
                                         {to_node_(*this), to_node_(dout)}, shape_));
  else
    return clone<float>().sigmoid_backward(dout);
}

template <value_type T>
inline array<float> array<T>::linear_sigmoid(const array &W, const array &b) const {
  if constexpr (std::is_same_v<T, float>) {
    if (dimension() != 2 || W.dimension() != 2 || shape_[1] != W.shape_[0])
      throw std::runtime_error("array: can't do `linear` operation.");
    return from_node_(detail::node::make(detail::op::linear_sigmoid,
                                         {to_node_(*this), to_node_(W), to_node_(b)},
                                         {shape_[0], W.shape_[1]}));
  } else {
    return linear(W, b).sigmoid();
  }
}

template <value_type T>
inline array<float> array<T>::relu() const {
  if constexpr (std::is_same_v<T, float>)
    return from_node_(detail::node::make(detail::op::relu, {to_node_(*this)}, shape_));
  else
    return clone<float>().relu();
}

template <value_type T>
inline array<float> array<T>::conv2d(const array<float> &weight, size_t kernel_size) const {
  if (dimension() != 4 || weight.dimension() != 4)
    throw std::runtime_error("array: conv2d requires a 4D NHWC input and a 4D OHWI weight.");
  const auto &ws = weight.shape();
  if (ws[1] != kernel_size || ws[2] != kernel_size || ws[3] != shape_[3] || kernel_size == 0)
    throw std::runtime_error("array: conv2d weight shape does not match the input.");
  if constexpr (std::is_same_v<T, float>) {
    auto n = detail::node::make(detail::op::conv2d, {to_node_(*this), to_node_(weight)},
                                shape_type{shape_[0], shape_[1], shape_[2], ws[0]});
    n->ksize = kernel_size;
    return from_node_(std::move(n));
  } else {
    return clone<float>().conv2d(weight, kernel_size);
  }
}

template <value_type T>
inline array<float> array<T>::layer_norm(const array<float> &gamma, const array<float> &beta,
                                         float eps) const {
  if (dimension() != 2) throw std::runtime_error("array: layer_norm requires 2D array.");
  // The kernel reads gamma[c] and beta[c] for every column c: shorter
  // vectors would be read past their end (the reference does not check).
  if (gamma.element_count() != shape_[1] || beta.element_count() != shape_[1])
    throw std::runtime_error("array: layer_norm needs one gamma and one beta per column.");
  if constexpr (std::is_same_v<T, float>) {
    auto n = detail::node::make(detail::op::layer_norm,
                                {to_node_(*this), to_node_(gamma), to_node_(beta)}, shape_);
    n->eps = eps;
    return from_node_(std::move(n));
  } else {
    return clone<float>().layer_norm(gamma, beta, eps);
  }
}

template <value_type T>
inline array<float> array<T>::softmax() const {
  if (dimension() != 1 && dimension() != 2)
    throw std::runtime_error("array: softmax is available only for 1 or 2 dimension array.");
  if constexpr (std::is_same_v<T, float>) {
    // A vector is one row (the reference computes this case on the host,
    // include/array.h:1678-1685).
    return from_node_(detail::node::make(detail::op::softmax, {to_node_(*this)}, shape_));
  } else {
    return clone<float>().softmax();
  }
}

template <value_type T>
inline array<T> array<T>::sum(size_t axis) const {
  if (axis >= dimension()) throw std::runtime_error("array: invalid axis.");
  auto s = shape_;
  s.erase(s.begin() + axis);
  if constexpr (std::is_same_v<T, float>) {
    auto n = detail::node::make(detail::op::sum_axis, {to_node_(*this)}, s);
    n->axis = axis;
    return from_node_(std::move(n));
  } else {
    array tmp(s, T{});
    std::vector<size_t> pos(dimension()), p2;
    for (size_t i = 0; i < element_count(); i++) {
      size_t r = i;
      for (size_t d = dimension(); d-- > 0;) {
        pos[d] = r % shape_[d];
        r /= shape_[d];
      }
      p2 = pos;
      p2.erase(p2.begin() + axis);
      tmp.at(p2) += at(pos);
    }
    return tmp;
  }
}

template <value_type T>
inline array<float> array<T>::mean(size_t axis) const {
  if constexpr (std::is_same_v<T, float>)
    return sum(axis) / array<float>(static_cast<float>(shape_[axis]));
  else
    return sum(axis).template clone<float>() / array<float>(static_cast<float>(shape_[axis]));
}

// Full reductions return a host value: the device reduces to one float and
// the host reads it (one 4-byte download instead of the reference's partials).
template <value_type T>
inline T array<T>::sum() const {
  if constexpr (std::is_same_v<T, float>) {
    require_gpu_();
    ensure_evaluated_();
    auto src = (is_contiguous_() && storage_.len >= element_count()) ? *this : materialize_();
    auto out = array<float>::make_uninit_({});
    gpu::sum_f32(src.storage_, out.storage_, src.element_count());
    return *out.storage_.template host_in<float>();
  } else {
    T s{};
    for (size_t i = 0; i < element_count(); i++) s += at(i);
    return s;
  }
}

template <value_type T>
inline T array<T>::min() const {
  if constexpr (std::is_same_v<T, float>) {
    require_gpu_();
    if (element_count() == 0) throw std::runtime_error("array: min of an empty array.");
    ensure_evaluated_();
    auto src = (is_contiguous_() && storage_.len >= element_count()) ? *this : materialize_();
    auto out = array<float>::make_uninit_({});
    gpu::min_f32(src.storage_, out.storage_, src.element_count());
    return *out.storage_.template host_in<float>();
  } else {
    T m = at(0);
    for (size_t i = 1; i < element_count(); i++) m = std::min(m, at(i));
    return m;
  }
}

template <value_type T>
inline T array<T>::max() const {
  if constexpr (std::is_same_v<T, float>) {
    require_gpu_();
    if (element_count() == 0) throw std::runtime_error("array: max of an empty array.");
    ensure_evaluated_();
    auto src = (is_contiguous_() && storage_.len >= element_count()) ? *this : materialize_();
    auto out = array<float>::make_uninit_({});
    gpu::max_f32(src.storage_, out.storage_, src.element_count());
    return *out.storage_.template host_in<float>();
  } else {
    T m = at(0);
    for (size_t i = 1; i < element_count(); i++) m = std::max(m, at(i));
    return m;
  }
}

// Per-row argmax of a 2-D array, first index of the maximum
// (include/array.h:1711-1750).  The float result stays on the device.
template <value_type T>
inline array<int> array<T>::argmax() const {
  if (dimension() != 2)
    throw std::runtime_error("array: argmax is available for 2 dimension array.");
  const size_t rows = shape_[0], cols = shape_[1];
  if constexpr (std::is_same_v<T, float>) {
    require_gpu_();
    auto src = is_contiguous_() ? *this : materialize_();
    src.ensure_evaluated_();
    auto out = array<int>::make_uninit_({rows});
    gpu::argmax_f32(src.storage_, out.storage_, uint32_t(rows), uint32_t(cols));
    return out;
  } else {
    array<int> out({rows}, 0);
    for (size_t r = 0; r < rows; r++) {
      size_t best = 0;
      for (size_t c = 1; c < cols; c++)
        if ((*this)[r, c] > (*this)[r, best]) best = c;
      out.at(r) = static_cast<int>(best);
    }
    return out;
  }
}

//------------------------------------------------------------------------------
// Free functions (include/array.h:2730-2831)
//------------------------------------------------------------------------------

template <value_type T>
inline std::ostream &operator<<(std::ostream &os, const array<T> &arr) {
  return os << arr.print_array();
}

template <value_type T>
inline array<T> operator+(arithmetic auto lhs, const array<T> &rhs) {
  return array<T>(static_cast<T>(lhs)) + rhs;
}
template <value_type T>
inline array<T> operator-(arithmetic auto lhs, const array<T> &rhs) {
  return array<T>(static_cast<T>(lhs)) - rhs;
}
template <value_type T>
inline array<T> operator*(arithmetic auto lhs, const array<T> &rhs) {
  return array<T>(static_cast<T>(lhs)) * rhs;
}
template <value_type T>
inline array<T> operator/(arithmetic auto lhs, const array<T> &rhs) {
  return array<T>(static_cast<T>(lhs)) / rhs;
}
template <value_type T>
inline array<T> operator+(const array<T> &lhs, arithmetic auto rhs) {
  return lhs + array<T>(static_cast<T>(rhs));
}
template <value_type T>
inline array<T> operator-(const array<T> &lhs, arithmetic auto rhs) {
  return lhs - array<T>(static_cast<T>(rhs));
}
template <value_type T>
inline array<T> operator*(const array<T> &lhs, arithmetic auto rhs) {
  return lhs * array<T>(static_cast<T>(rhs));
}
template <value_type T>
inline array<T> operator/(const array<T> &lhs, arithmetic auto rhs) {
  return lhs / array<T>(static_cast<T>(rhs));
}

template <value_type T, value_type U>
inline array<T> where(const array<U> &cond, T x, T y) {
  array<T> tmp(cond.shape(), T{});
  for (size_t i = 0; i < cond.element_count(); i++) tmp.at(i) = cond.at(i) ? x : y;
  return tmp;
}

template <value_type T>
inline bool array_equal(const array<T> &a, const array<T> &b) {
  if (&a == &b) return true;
  if (a.shape() != b.shape()) return false;
  for (size_t i = 0; i < a.element_count(); i++)
    if (a.at(i) != b.at(i)) return false;
  return true;
}

template <std::floating_point T, std::floating_point U>
inline bool is_close(T a, U b, float tolerance = 1e-3) {
  return std::abs(static_cast<float>(a) - static_cast<float>(b)) <= tolerance;
}
template <std::integral T, std::integral U>
inline bool is_close(T a, U b) {
  return a == b;
}

template <value_type T>
inline bool allclose(const array<T> &a, const array<T> &b, float tolerance = 1e-3) {
  if (&a == &b) return true;
  if (a.shape() != b.shape()) return false;
  for (size_t i = 0; i < a.element_count(); i++) {
    if constexpr (std::is_same_v<T, float>) {
      if (std::abs(a.at(i) - b.at(i)) > tolerance) return false;
    } else {
      if (a.at(i) != b.at(i)) return false;
    }
  }
  return true;
}

template <value_type T>
inline auto empty(const shape_type &shape) {
  return array<T>(shape, T{});
}
template <value_type T>
inline auto zeros(const shape_type &shape) {
  return array<T>(shape, T(0));
}
template <value_type T>
inline auto ones(const shape_type &shape) {
  return array<T>(shape, T(1));
}
inline auto random(const shape_type &shape) {
  array<float> tmp(shape, 0.0f);
  tmp.random();
  return tmp;
}

// Evaluates several arrays' graphs in one pass and waits for the GPU
// (include/array.h:2836-2888).
template <value_type... Ts>
inline void eval(array<Ts> &...arrays) {
  std::vector<detail::node *> roots;
  auto collect = [&](auto &arr) {
    auto n = arr.lazy_node_ptr();
    if (n && !n->evaluated) roots.push_back(n.get());
  };
  (collect(arrays), ...);
  if (!roots.empty()) detail::evaluate(roots);
  if (gpu_pending_) gpu_context::instance().flush();
  (arrays.eval(), ...);
}

//------------------------------------------------------------------------------
// Graph evaluation
//------------------------------------------------------------------------------

namespace detail {

// Host value of a length-1 operand, if it can be read without waiting for
// the GPU (a host-written scalar); std::nullopt otherwise.
inline bool host_scalar(const node *n, float &v) {
  if (!n->evaluated || n->data.len != 1) return false;
  auto *b = n->data.buf.get();
  if (!b->host || !b->host_valid) return false;
  v = static_cast<const float *>(b->host)[n->data.off];
  return true;
}

struct program_builder {
  silgpu_program p{};
  shape_type out_shape;
  std::vector<storage> keep;  // inputs kept alive until launch
  std::vector<std::tuple<const void *, strides_type>> slots;
  bool free_reg[SILGPU_PROG_MAX_REGS];
  const std::unordered_set<node *> *fused = nullptr;  // nodes computed inside this program

  struct too_big {};

  explicit program_builder(const shape_type &shape) : out_shape(shape) {
    if (shape.size() > SILGPU_PROG_MAX_DIMS) throw too_big{};
    p.ndim = static_cast<int32_t>(shape.size());
    for (size_t d = 0; d < shape.size(); d++) p.shape[d] = int64_t(shape[d]);
    std::fill(std::begin(free_reg), std::end(free_reg), true);
  }

  int alloc() {
    for (int r = 0; r < SILGPU_PROG_MAX_REGS; r++)
      if (free_reg[r]) {
        free_reg[r] = false;
        return r;
      }
    throw too_big{};
  }
  void release(int r) { free_reg[r] = true; }

  void emit(int32_t op, int32_t dst, int32_t a, int32_t b = 0, float imm = 0, float imm2 = 0) {
    if (p.n_instrs >= SILGPU_PROG_MAX_INSTRS) throw too_big{};
    p.instrs[p.n_instrs++] = silgpu_prog_instr{op, dst, a, b, imm, imm2};
  }

  // Input slot for an evaluated node, with strides relative to the output
  // shape (right-aligned broadcast; size-1 axes broadcast with stride 0).
  int slot(node *n) {
    const size_t no = out_shape.size(), ni = n->shape.size();
    strides_type st(no, 0);
    for (size_t d = 0; d < no; d++) {
      if (d + ni < no) continue;
      const size_t di = d + ni - no;
      st[d] = (n->shape[di] == 1 && out_shape[d] != 1) ? 0 : n->strides[di];
    }
    const void *ptr = n->data.template dev_in<float>();
    for (size_t i = 0; i < slots.size(); i++)
      if (std::get<0>(slots[i]) == ptr && std::get<1>(slots[i]) == st) return int(i);
    if (slots.size() >= SILGPU_PROG_MAX_INPUTS) throw too_big{};
    const int s = int(slots.size());
    slots.emplace_back(ptr, st);
    keep.push_back(n->data);
    p.inputs[s].ptr = static_cast<const float *>(ptr);
    for (size_t d = 0; d < no; d++) p.inputs[s].strides[d] = int64_t(st[d]);
    p.n_inputs = s + 1;
    return s;
  }

  // Sethi-Ullman register need of the fused subtree at n.
  int need(node *n) const {
    if (!fused->count(n)) return 1;
    if (n->operation == op::sigmoid || n->operation == op::relu || n->operation == op::copy)
      return need(n->inputs[0].get());
    int a = need(n->inputs[0].get()), b = need(n->inputs[1].get());
    return a == b ? a + 1 : std::max(a, b);
  }

  // Emits the value of n into a register and returns it.
  int value(node *n) {
    if (!fused->count(n)) {
      int r = alloc();
      emit(SILGPU_PI_LOAD, r, slot(n));
      return r;
    }
    const op o = n->operation;
    if (o == op::copy) return value(n->inputs[0].get());
    if (o == op::sigmoid || o == op::relu) {
      int r = value(n->inputs[0].get());
      emit(o == op::sigmoid ? SILGPU_PI_SIGMOID : SILGPU_PI_RELU, r, r);
      return r;
    }
    node *a = n->inputs[0].get(), *b = n->inputs[1].get();
    if (o == op::sigmoid_backward) {  // inputs {x, dout}
      auto [ra, rb] = pair_(a, b);
      emit(SILGPU_PI_SIGBWD, ra, ra, rb);
      release(rb);
      return ra;
    }
    // Scalar operand folded the way the reference's try_affine_reduce folds
    // one level per node (include/array.h:1888-1940): x op s and s op x
    // become fma(x, scale, offset) with scale/offset formed in fp32 on the
    // host, so the fused result is bit-identical to that evaluation.
    float s;
    if (o != op::pow && host_scalar(b, s) && !fused->count(b)) {
      int r = value(a);
      float scale = 1.0f, offset = 0.0f;
      switch (o) {
        case op::add: offset = 0.0f + s; break;
        case op::sub: offset = 0.0f - s; break;
        case op::mul: scale = 1.0f * s; offset = 0.0f * s; break;
        default: scale = 1.0f / s; offset = 0.0f / s; break;  // div
      }
      emit(SILGPU_PI_FMAI, r, r, 0, scale, offset);
      return r;
    }
    if (o != op::pow && o != op::div && host_scalar(a, s) && !fused->count(a)) {
      int r = value(b);
      float scale = 1.0f, offset = 0.0f;
      switch (o) {
        case op::add: offset = 0.0f + s; break;
        case op::sub: scale = -1.0f; offset = s - 0.0f; break;
        default: scale = 1.0f * s; offset = 0.0f * s; break;  // mul
      }
      emit(SILGPU_PI_FMAI, r, r, 0, scale, offset);
      return r;
    }
    auto [ra, rb] = pair_(a, b);
    const int32_t code = o == op::add ? SILGPU_PI_ADD : o == op::sub ? SILGPU_PI_SUB
                         : o == op::mul ? SILGPU_PI_MUL : o == op::div ? SILGPU_PI_DIV
                                                                        : SILGPU_PI_POW;
    emit(code, ra, ra, rb);
    release(rb);
    return ra;
  }

  // Both operands in registers, the subtree needing more registers first.
  std::pair<int, int> pair_(node *a, node *b) {
    if (need(b) > need(a)) {
      int rb = value(b);
      int ra = value(a);
      return {ra, rb};
    }
    int ra = value(a);
    int rb = value(b);
    return {ra, rb};
  }
};

inline storage new_output(const shape_type &shape) {
  auto s = storage::make_device(shape_count(shape) * sizeof(float));
  s.len = shape_count(shape);
  return s;
}

inline void finish(node *n, storage out) {
  n->data = std::move(out);
  n->strides = contiguous_strides(n->shape);
  n->evaluated = true;
}

inline array<float> as_array(node *n) { return array<float>::view_(n->data, n->shape, n->strides); }

// The storage of an evaluated node as a contiguous float array (copies
// strided or broadcast views).
inline array<float> contiguous(node *n) {
  auto a = as_array(n);
  a.eval();
  if (a.is_contiguous_() && n->data.len >= shape_count(n->shape)) return a;
  return a.materialize_();
}

// 2-D operand of a product: (storage, leading dimension, transposed?) for a
// view whose inner axis is unit-stride (row-major) or whose outer axis is
// (a transposed view); anything else is copied first.
struct gemm_operand {
  array<float> arr;
  size_t ld = 0;
  bool trans = false;
};

inline gemm_operand operand2d(node *n, const shape_type &as2d) {
  auto a = as_array(n);
  a.eval();
  if (n->shape.size() == 2) {
    const auto &st = n->strides;
    if (st[1] == 1 && st[0] >= n->shape[1] && st[0] > 0) return {a, st[0], false};
    if (st[0] == 1 && st[1] >= n->shape[0] && st[1] > 0) return {a, st[1], true};
  }
  auto c = a.is_contiguous_() ? a : a.materialize_();
  return {c, as2d[1], false};
}

// Descriptor of a single (batch 1) product with n's fused scale.
inline silgpu_gemm_desc product_desc(size_t M, size_t N, size_t K, const gemm_operand &A,
                                     const gemm_operand &B, size_t ldc, const node *n) {
  silgpu_gemm_desc d{};
  d.trans_a = A.trans;
  d.trans_b = B.trans;
  d.M = int64_t(M);
  d.N = int64_t(N);
  d.K = int64_t(K);
  d.lda = int64_t(A.ld);
  d.ldb = int64_t(B.ld);
  d.ldc = int64_t(ldc);
  d.batch_outer = d.batch_inner = 1;
  d.epilogue = SILGPU_EPI_NONE;
  d.use_scale = n->use_scale;
  d.scale = n->scale;
  d.scale_offset = n->scale_offset;
  return d;
}

// The residual operand fused into n's epilogue (a 2-D view with unit column
// stride, already evaluated), kept alive in `keep` until the launch.
inline void add_residual(silgpu_gemm_desc &d, const node *n, std::optional<array<float>> &keep) {
  if (!n->residual) return;
  node *x = n->residual.get();
  if (!x->evaluated) throw std::runtime_error("array: residual operand not evaluated.");
  keep = as_array(x);
  d.ldr = int64_t(x->strides[0]);
}

inline void eval_dot(node *n) {
  node *l = n->inputs[0].get(), *r = n->inputs[1].get();
  // 1-D operands: v . m -> {1,K}.{K,N}; m . v -> {M,K}.{K,1}; v . v -> {1,K}.{K,1}
  // (include/array.h:2700-2728).
  const bool lv = l->shape.size() == 1, rv = r->shape.size() == 1;
  const size_t M = lv ? 1 : l->shape[0], K = lv ? l->shape[0] : l->shape[1];
  const size_t N = rv ? 1 : r->shape[1];
  gemm_operand A, B;
  if (lv) {
    auto c = contiguous(l);
    A = {c, K, false};
  } else {
    A = operand2d(l, {M, K});
  }
  if (rv) {
    auto c = contiguous(r);
    B = {c, 1, false};  // K x 1, ld 1
  } else {
    B = operand2d(r, {K, N});
  }
  auto out = new_output(n->shape);
  auto d = product_desc(M, N, K, A, B, N, n);
  std::optional<array<float>> res;
  add_residual(d, n, res);
  gpu::gemm(d, A.arr.storage_ref(), B.arr.storage_ref(), out, nullptr,
            res ? &res->storage_ref() : nullptr);
  finish(n, std::move(out));
}

inline void eval_linear(node *n, bool with_sigmoid) {
  node *x = n->inputs[0].get(), *w = n->inputs[1].get(), *b = n->inputs[2].get();
  const size_t M = x->shape[0], K = x->shape[1], N = w->shape[1];
  auto A = operand2d(x, {M, K});
  auto B = operand2d(w, {K, N});
  auto out = new_output(n->shape);
  const size_t bl = shape_count(b->shape);
  if (b->shape.size() <= 1 && bl > 0) {
    // Bias read as bias[col % bias_len] in the GEMM epilogue
    // (include/gpu_kernels.metal:506-542).
    auto bias = contiguous(b);
    auto d = product_desc(M, N, K, A, B, N, n);
    d.epilogue = with_sigmoid ? SILGPU_EPI_BIAS_SIGMOID
                 : n->epilogue == SILGPU_EPI_BIAS_RELU ? SILGPU_EPI_BIAS_RELU
                                                        : SILGPU_EPI_BIAS;
    d.bias_len = int64_t(bl);
    std::optional<array<float>> res;
    add_residual(d, n, res);
    gpu::gemm(d, A.arr.storage_ref(), B.arr.storage_ref(), out, &bias.storage_ref(),
              res ? &res->storage_ref() : nullptr);
    finish(n, std::move(out));
    return;
  }
  // Higher-rank bias: product, then a broadcast add (and sigmoid) program.
  gpu::gemm_(A.arr.storage_ref(), B.arr.storage_ref(), out, M, N, K, A.ld, B.ld, A.trans,
             B.trans, 1, 0, 0, 0, nullptr, 0, SILGPU_EPI_NONE);
  auto prod = node::leaf(out, n->shape, contiguous_strides(n->shape));
  std::unordered_set<node *> none;
  program_builder pb(n->shape);
  pb.fused = &none;
  int r = pb.alloc();
  pb.emit(SILGPU_PI_LOAD, r, pb.slot(prod.get()));
  int rb = pb.alloc();
  pb.emit(SILGPU_PI_LOAD, rb, pb.slot(b));
  pb.emit(SILGPU_PI_ADD, r, r, rb);
  if (with_sigmoid) pb.emit(SILGPU_PI_SIGMOID, r, r);
  if (n->epilogue == SILGPU_EPI_BIAS_RELU) pb.emit(SILGPU_PI_RELU, r, r);
  pb.p.out_reg = r;
  auto res = new_output(n->shape);
  gpu::program(pb.p, res);
  finish(n, std::move(res));
}

// Matrix layout of the last two axes of an operand view: row-major with
// leading dimension ld, or transposed (column-major) with leading dimension
// ld; false if neither (the operand is then copied).
inline bool mat_layout(const node *x, size_t rows, size_t cols, size_t &ld, bool &trans) {
  const size_t nd = x->shape.size();
  const size_t sr = x->strides[nd - 2], sc = x->strides[nd - 1];
  if ((sc == 1 || cols == 1) && sr >= cols && sr > 0) {
    ld = sr;
    trans = false;
    return true;
  }
  if ((sr == 1 || rows == 1) && sc >= rows && sc > 0) {
    ld = sc;
    trans = true;
    return true;
  }
  return false;
}

// {..., M, K} x {..., K, N}.  The leading axes that both operands stride
// uniformly become one batched launch; the rest are looped over.
inline void eval_batched(node *n) {
  node *l = n->inputs[0].get(), *r = n->inputs[1].get();
  const size_t nd = n->shape.size(), L = nd - 2;
  const size_t M = n->shape[nd - 2], N = n->shape[nd - 1], K = l->shape[nd - 1];
  std::shared_ptr<node> lc, rc;  // contiguous copies when a layout is not usable
  size_t lda, ldb;
  bool ta, tb;
  if (!mat_layout(l, M, K, lda, ta)) {
    auto c = contiguous(l);
    lc = node::leaf(c.storage_ref(), l->shape, contiguous_strides(l->shape));
    l = lc.get();
    mat_layout(l, M, K, lda, ta);
  }
  if (!mat_layout(r, K, N, ldb, tb)) {
    auto c = contiguous(r);
    rc = node::leaf(c.storage_ref(), r->shape, contiguous_strides(r->shape));
    r = rc.get();
    mat_layout(r, K, N, ldb, tb);
  }
  // Fold the leading axes into at most two batch groups, each a run of
  // axes that both operands stride uniformly (stride[d] == stride[d+1] *
  // extent[d+1]): [inner, L) is the inner batch, [outer_begin, inner) the
  // outer one; any axes left before outer_begin are looped over.  A
  // [batch, heads, seq, dim] view split out of one [batch*seq, 3*heads*dim]
  // array is one launch: heads are the inner group, batches the outer.
  // C's strides: contiguous, or the reordered layout the lowering chose.
  const strides_type cs = n->out_strides.empty() ? contiguous_strides(n->shape) : n->out_strides;
  auto uniform = [&](size_t d) {
    return l->strides[d] == l->strides[d + 1] * l->shape[d + 1] &&
           r->strides[d] == r->strides[d + 1] * r->shape[d + 1] &&
           cs[d] == cs[d + 1] * n->shape[d + 1];
  };
  size_t inner = L, outer_begin = L;
  size_t binner = 1, bouter = 1;
  if (L > 0) {
    inner = L - 1;
    binner = n->shape[L - 1];
    while (inner > 0 && uniform(inner - 1)) binner *= n->shape[--inner];
    outer_begin = inner;
    if (inner > 0) {
      outer_begin = inner - 1;
      bouter = n->shape[inner - 1];
      while (outer_begin > 0 && uniform(outer_begin - 1)) bouter *= n->shape[--outer_begin];
    }
  }
  silgpu_gemm_desc d{};
  d.trans_a = ta;
  d.trans_b = tb;
  d.M = int64_t(M);
  d.N = int64_t(N);
  d.K = int64_t(K);
  d.lda = int64_t(lda);
  d.ldb = int64_t(ldb);
  d.ldc = int64_t(cs[nd - 2]);
  d.batch_outer = int64_t(bouter);
  d.batch_inner = int64_t(binner);
  d.stride_a_inner = L > 0 ? int64_t(l->strides[L - 1]) : 0;
  d.stride_b_inner = L > 0 ? int64_t(r->strides[L - 1]) : 0;
  d.stride_c_inner = L > 0 ? int64_t(cs[L - 1]) : 0;
  d.stride_a_outer = inner > 0 ? int64_t(l->strides[inner - 1]) : 0;
  d.stride_b_outer = inner > 0 ? int64_t(r->strides[inner - 1]) : 0;
  d.stride_c_outer = inner > 0 ? int64_t(cs[inner - 1]) : 0;
  d.epilogue = SILGPU_EPI_NONE;
  d.use_scale = n->use_scale;
  d.scale = n->scale;
  d.scale_offset = n->scale_offset;
  auto out = new_output(n->shape);
  size_t loops = 1;
  for (size_t a = 0; a < outer_begin; a++) loops *= n->shape[a];
  for (size_t o = 0; o < loops; o++) {
    size_t rem = o, offa = 0, offb = 0, offc = 0;
    for (size_t a = outer_begin; a-- > 0;) {
      const size_t idx = rem % n->shape[a];
      rem /= n->shape[a];
      offa += idx * l->strides[a];
      offb += idx * r->strides[a];
      offc += idx * cs[a];
    }
    storage A = l->data, B = r->data, C = out;
    A.off += offa;
    B.off += offb;
    C.off += offc;
    C.len = out.len - offc;
    gpu::gemm(d, A, B, C);
  }
  finish(n, std::move(out));
  n->strides = cs;
}

// Folds the leading `L` axes of `shape` into at most two groups that every
// operand strides uniformly (stride[d] == stride[d+1] * shape[d+1]): the
// inner group [inner, L) and the outer [0, inner).  False when the axes
// need more groups.
inline bool fold_two_groups(const shape_type &shape, size_t L,
                            const std::vector<const strides_type *> &ops, int64_t &bo,
                            int64_t &bi, std::vector<std::pair<int64_t, int64_t>> &st) {
  bo = bi = 1;
  st.assign(ops.size(), {0, 0});
  if (L == 0) return true;
  auto uniform = [&](size_t d) {
    for (const strides_type *s : ops)
      if ((*s)[d] != (*s)[d + 1] * shape[d + 1]) return false;
    return true;
  };
  size_t inner = L - 1;
  bi = int64_t(shape[L - 1]);
  while (inner > 0 && uniform(inner - 1)) bi *= int64_t(shape[--inner]);
  if (inner > 0) {
    size_t outer = inner - 1;
    bo = int64_t(shape[outer]);
    while (outer > 0 && uniform(outer - 1)) bo *= int64_t(shape[--outer]);
    if (outer > 0) return false;
  }
  for (size_t i = 0; i < ops.size(); i++)
    st[i] = {inner > 0 ? int64_t((*ops[i])[inner - 1]) : 0, int64_t((*ops[i])[L - 1])};
  return true;
}

// A fused attention launch: n = batched_dot(softmax(q k^T * scale), v).
struct attention_plan {
  node *q = nullptr, *kt = nullptr, *v = nullptr;
  float scale = 1.0f;
  silgpu_attn_desc desc{};  // extents, leading dimensions and batch strides
};

inline void eval_attention(node *n, const attention_plan &p) {
  auto out = new_output(n->shape);
  gpu::attention(p.desc, p.q->data, p.kt->data, p.v->data, out);
  finish(n, std::move(out));
  if (!n->out_strides.empty()) n->strides = n->out_strides;
}

inline void eval_node_nonfused(node *n) {
  switch (n->operation) {
    case op::dot:
      eval_dot(n);
      return;
    case op::batched_dot:
      eval_batched(n);
      return;
    case op::view: {
      node *src = n->inputs[0].get();
      storage v = src->data;
      v.off = src->data.off + n->view_off;
      size_t span = 1;
      for (size_t d = 0; d < n->shape.size(); d++)
        if (n->shape[d] > 0) span += (n->shape[d] - 1) * n->strides[d];
      v.len = shape_count(n->shape) == 0 ? 0 : span;
      n->data = v;
      n->evaluated = true;  // shape and strides are the view's own
      return;
    }
    case op::linear:
      eval_linear(n, false);
      return;
    case op::linear_sigmoid:
      eval_linear(n, true);
      return;
    case op::softmax: {
      auto a = contiguous(n->inputs[0].get());
      auto out = new_output(n->shape);
      const size_t rows = n->shape.size() == 2 ? n->shape[0] : 1;
      gpu::softmax(a.storage_ref(), out, uint32_t(rows), uint32_t(n->shape.back()));
      finish(n, std::move(out));
      return;
    }
    case op::conv2d: {
      auto x = contiguous(n->inputs[0].get());
      auto w = contiguous(n->inputs[1].get());
      const auto &xs = n->inputs[0]->shape;
      auto out = new_output(n->shape);
      gpu::conv2d(x.storage_ref(), w.storage_ref(), out, uint32_t(xs[0]), uint32_t(xs[1]),
                  uint32_t(xs[2]), uint32_t(xs[3]), uint32_t(n->ksize), uint32_t(n->shape[3]));
      finish(n, std::move(out));
      return;
    }
    case op::layer_norm: {
      auto a = contiguous(n->inputs[0].get());
      auto g = contiguous(n->inputs[1].get());
      auto b = contiguous(n->inputs[2].get());
      const size_t cols = n->shape[1];
      if (g.element_count() < cols || b.element_count() < cols)
        throw std::runtime_error("array: layer_norm gamma/beta shorter than the rows.");
      auto out = new_output(n->shape);
      gpu::layer_norm(a.storage_ref(), out, g.storage_ref(), b.storage_ref(),
                      uint32_t(n->shape[0]), uint32_t(cols), n->eps);
      finish(n, std::move(out));
      return;
    }
    case op::sum_axis: {
      node *in = n->inputs[0].get();
      auto a = contiguous(in);
      size_t outer = 1, inner = 1;
      for (size_t d = 0; d < n->axis; d++) outer *= in->shape[d];
      for (size_t d = n->axis + 1; d < in->shape.size(); d++) inner *= in->shape[d];
      auto out = new_output(n->shape);
      gpu::sum_axis(a.storage_ref(), out, outer, in->shape[n->axis], inner);
      finish(n, std::move(out));
      return;
    }
    default:
      throw std::runtime_error("array: unsupported lazy operation.");
  }
}

// Runs the fused program for elementwise root n over the subtree in `fused`.
inline bool try_program(node *n, const std::unordered_set<node *> &fused) {
  try {
    program_builder pb(n->shape);
    pb.fused = &fused;
    int r = pb.value(n);
    pb.p.out_reg = r;
    auto out = new_output(n->shape);
    if (shape_count(n->shape) > 0) gpu::program(pb.p, out);
    finish(n, std::move(out));
    return true;
  } catch (program_builder::too_big &) {
    return false;
  }
}

inline void evaluate(const std::vector<node *> &roots) {
  if (device_ == Device::CPU)
    throw std::runtime_error(
        "array: float evaluation needs the GPU backend (sil::use_gpu()); the CPU backend "
        "is not part of this build.");
  // Post-order DFS over unevaluated nodes (include/array.h:1945-1971).
  std::vector<node *> order;
  std::unordered_set<node *> seen;
  // Each root's traversal completes before the next root starts, so a root
  // that another root consumes is ordered before its consumer.
  std::vector<std::pair<node *, uint8_t>> stack;
  for (node *r : roots) {
    if (!r || r->evaluated || !seen.insert(r).second) continue;
    stack.push_back({r, 0});
    while (!stack.empty()) {
      auto &[cur, idx] = stack.back();
      if (idx < cur->num_inputs) {
        node *c = cur->inputs[idx++].get();
        if (c && !c->evaluated && seen.insert(c).second) stack.push_back({c, 0});
      } else {
        order.push_back(cur);
        stack.pop_back();
      }
    }
  }
  // Consumers inside this graph, and the single consumer where there is one.
  std::unordered_map<node *, int> consumers;
  std::unordered_map<node *, node *> parent;
  for (node *n : order)
    for (uint8_t i = 0; i < n->num_inputs; i++) {
      node *c = n->inputs[i].get();
      if (!c->evaluated) {
        consumers[c]++;
        parent[c] = n;
      }
    }
  const std::unordered_set<node *> root_set(roots.begin(), roots.end());
  std::unordered_map<node *, size_t> pos;
  for (size_t i = 0; i < order.size(); i++) pos[order[i]] = i;
  // c is consumed only by p inside this graph, is not requested itself and
  // no array outside the graph holds it.
  auto single_use = [&](node *c, node *p) {
    if (c->evaluated || root_set.count(c)) return false;
    auto it = consumers.find(c);
    if (it == consumers.end() || it->second != 1) return false;
    for (uint8_t i = 0; i < p->num_inputs; i++)
      if (p->inputs[i].get() == c) return p->inputs[i].use_count() == 1;
    return false;
  };
  auto bias_vector = [](node *lin) {
    node *b = lin->inputs[2].get();
    return shape_count(b->shape) > 0 && b->shape.size() <= 1;
  };
  // Nodes whose result is another node's output (alias[n]): the lowering
  // folds them into the epilogue of the product they consume.
  std::unordered_map<node *, node *> alias;
  std::unordered_set<node *> materialize;  // operands a fused epilogue reads
  //  relu(linear(x, W, b)): the relu runs in the GEMM epilogue.
  for (node *n : order) {
    if (n->operation != op::relu) continue;
    node *c = n->inputs[0].get();
    if (c->operation != op::linear || !single_use(c, n) || !bias_vector(c)) continue;
    c->epilogue = SILGPU_EPI_BIAS_RELU;
    alias[n] = c;
  }
  //  product op host-scalar (and scalar op product): the node's fmaf runs in
  //  the epilogue of dot / batched_dot, with the scale and offset the
  //  program builder would use, so the result is bit-identical.
  for (node *n : order) {
    if (!is_binary(n->operation) || n->operation == op::pow) continue;
    node *a = n->inputs[0].get(), *b = n->inputs[1].get();
    auto is_product = [](node *x) {
      return x->operation == op::dot || x->operation == op::batched_dot;
    };
    float s = 0.0f, scale = 1.0f, offset = 0.0f;
    node *c = nullptr;
    if (is_product(a) && host_scalar(b, s)) {
      c = a;
      switch (n->operation) {
        case op::add: offset = 0.0f + s; break;
        case op::sub: offset = 0.0f - s; break;
        case op::mul: scale = 1.0f * s; offset = 0.0f * s; break;
        default: scale = 1.0f / s; offset = 0.0f / s; break;  // div
      }
    } else if (n->operation != op::div && is_product(b) && host_scalar(a, s)) {
      c = b;
      switch (n->operation) {
        case op::add: offset = 0.0f + s; break;
        case op::sub: scale = -1.0f; offset = s - 0.0f; break;
        default: scale = 1.0f * s; offset = 0.0f * s; break;  // mul
      }
    }
    if (!c || c->use_scale || c->shape != n->shape || !single_use(c, n)) continue;
    c->use_scale = true;
    c->scale = scale;
    c->scale_offset = offset;
    alias[n] = c;
  }
  //  x + product (either side): the add runs after the product's epilogue,
  //  reading x (a 2-D array with unit column stride computed before the
  //  product) as the residual.
  for (node *n : order) {
    if (n->operation != op::add || alias.count(n) || n->shape.size() != 2) continue;
    for (int side = 0; side < 2; side++) {
      node *p = n->inputs[side].get(), *x = n->inputs[1 - side].get();
      node *c = alias.count(p) ? alias[p] : p;
      // A product evaluated earlier (a view of it forced it, or an earlier
      // eval) has released its inputs: nothing to fuse, and its operands
      // must not be read.
      if (c->evaluated) continue;
      const bool ok_op = (c->operation == op::dot && c->inputs[0]->shape.size() == 2 &&
                          c->inputs[1]->shape.size() == 2) ||
                         ((c->operation == op::linear || c->operation == op::linear_sigmoid) &&
                          bias_vector(c));
      if (!ok_op || c->evaluated || c->residual || c->shape != n->shape) continue;
      if (!single_use(p, n) || x == c || x->shape != n->shape) continue;
      if (x->strides.size() != 2 || x->strides[1] != 1 || x->strides[0] < n->shape[1]) continue;
      if (!x->evaluated && !(pos.count(x) && pos.count(c) && pos[x] < pos[c])) continue;
      c->residual = n->inputs[1 - side];
      materialize.insert(x);
      alias[n] = c;
      break;
    }
  }
  //  copy(view(batched_dot)) where the view only reorders the product's
  //  axes and keeps its last one (attention's head merge,
  //  ctx.permute({0, 2, 1, 3}) before a reshape): the product writes its
  //  tiles straight into the copy's contiguous layout through ldc and batch
  //  strides, and the copy and the view alias its output.
  std::unordered_map<node *, node *> relayout;  // copy or view -> product
  for (node *n : order) {
    if (n->operation != op::copy || alias.count(n)) continue;
    node *v = n->inputs[0].get();
    if (v->operation != op::view || v->view_off != 0 || !single_use(v, n)) continue;
    node *p = v->inputs[0].get();
    if (p->operation != op::batched_dot || p->residual || !p->out_strides.empty()) continue;
    if (!single_use(p, v) || v->shape.size() != p->shape.size()) continue;
    const size_t nd = p->shape.size();
    const auto ps = contiguous_strides(p->shape), ns = contiguous_strides(v->shape);
    // perm[a] = the product axis that view axis a reads.
    std::vector<size_t> perm(nd, nd);
    bool ok = shape_count(p->shape) > 0;
    std::vector<bool> used(nd, false);
    for (size_t a = 0; ok && a < nd; a++) {
      for (size_t b = 0; b < nd; b++)
        if (!used[b] && ps[b] == v->strides[a] && p->shape[b] == v->shape[a] &&
            (p->shape[b] > 1 || v->strides[a] == ps[b])) {
          perm[a] = b;
          used[b] = true;
          break;
        }
      ok = perm[a] < nd;
    }
    if (!ok || perm[nd - 1] != nd - 1) continue;  // the product's rows stay unit-stride
    strides_type os(nd);
    for (size_t a = 0; a < nd; a++) os[perm[a]] = ns[a];
    p->out_strides = os;
    relayout[v] = p;
    relayout[n] = p;
  }
  //  batched_dot(view?(softmax(view?(S))), v) with S = batched_dot(q, k^T)
  //  (its scalar scale folded above) and the scores used by nothing else:
  //  one fused attention launch, the scores never stored
  //  (silgpu_attention_f32).  Needs unit stride along the head dim of q,
  //  k and v, a head dim of 16, 32, 64 or 128, and leading axes that fold
  //  into two uniformly strided batch groups.
  std::unordered_map<node *, attention_plan> attention;
  std::unordered_set<node *> attn_inner;  // nodes a fused attention computes
  auto plain_view = [](node *x) {
    return x->operation == op::view && x->view_off == 0 &&
           x->strides == contiguous_strides(x->shape);
  };
  for (node *n : order) {
    if (n->operation != op::batched_dot || n->use_scale || n->residual) continue;
    std::vector<node *> inner;
    node *prev = n, *cur = n->inputs[0].get();
    auto step = [&](node *next) {
      inner.push_back(cur);
      prev = cur;
      cur = next;
    };
    if (plain_view(cur)) {
      if (!single_use(cur, prev)) continue;
      step(cur->inputs[0].get());
    }
    if (cur->operation != op::softmax || cur->shape.size() != 2 || !single_use(cur, prev))
      continue;
    step(cur->inputs[0].get());
    if (plain_view(cur)) {
      if (!single_use(cur, prev)) continue;
      step(cur->inputs[0].get());
    }
    node *s1 = cur;
    if (auto it = alias.find(cur); it != alias.end()) {
      if (!single_use(cur, prev)) continue;
      s1 = it->second;
      step(s1);
    }
    if (s1->operation != op::batched_dot || s1->residual || !single_use(s1, prev)) continue;
    if (s1->use_scale && s1->scale_offset != 0.0f) continue;
    inner.push_back(s1);
    const size_t nd = n->shape.size();
    if (nd < 2 || s1->shape.size() != nd || inner.front()->shape != s1->shape) continue;
    node *q = s1->inputs[0].get(), *kt = s1->inputs[1].get(), *v = n->inputs[1].get();
    const size_t Sq = s1->shape[nd - 2], Sk = s1->shape[nd - 1], D = q->shape[nd - 1];
    if (n->shape[nd - 1] != D || (D != 16 && D != 32 && D != 64 && D != 128)) continue;
    if (q->strides[nd - 1] != 1 || kt->strides[nd - 2] != 1 || v->strides[nd - 1] != 1)
      continue;
    const strides_type cs =
        n->out_strides.empty() ? contiguous_strides(n->shape) : n->out_strides;
    const int64_t ldq = Sq > 1 ? int64_t(q->strides[nd - 2]) : int64_t(D);
    const int64_t ldk = Sk > 1 ? int64_t(kt->strides[nd - 1]) : int64_t(D);
    const int64_t ldv = Sk > 1 ? int64_t(v->strides[nd - 2]) : int64_t(D);
    const int64_t ldo = Sq > 1 ? int64_t(cs[nd - 2]) : int64_t(D);
    if (ldq < int64_t(D) || ldk < int64_t(D) || ldv < int64_t(D) || ldo < int64_t(D)) continue;
    attention_plan ap;
    std::vector<std::pair<int64_t, int64_t>> st;
    if (!fold_two_groups(n->shape, nd - 2, {&q->strides, &kt->strides, &v->strides, &cs},
                         ap.desc.batch_outer, ap.desc.batch_inner, st))
      continue;
    ap.q = q;
    ap.kt = kt;
    ap.v = v;
    ap.scale = s1->use_scale ? s1->scale : 1.0f;
    ap.desc.Sq = int64_t(Sq);
    ap.desc.Sk = int64_t(Sk);
    ap.desc.D = int64_t(D);
    ap.desc.scale = ap.scale;
    ap.desc.ldq = ldq;
    ap.desc.ldk = ldk;
    ap.desc.ldv = ldv;
    ap.desc.ldo = ldo;
    ap.desc.stride_q_outer = st[0].first;
    ap.desc.stride_q_inner = st[0].second;
    ap.desc.stride_k_outer = st[1].first;
    ap.desc.stride_k_inner = st[1].second;
    ap.desc.stride_v_outer = st[2].first;
    ap.desc.stride_v_inner = st[2].second;
    ap.desc.stride_o_outer = st[3].first;
    ap.desc.stride_o_inner = st[3].second;
    attention[n] = ap;
    for (node *x : inner) attn_inner.insert(x);
  }
  // A node is computed inside its consumer's program when it is elementwise,
  // has exactly one consumer, that consumer is elementwise, it is not a root
  // and no array outside the graph holds it.
  auto fusable = [&](node *c) {
    if (c->evaluated || root_set.count(c) || !is_elementwise(c->operation)) return false;
    if (materialize.count(c) || alias.count(c) || relayout.count(c) || attn_inner.count(c))
      return false;
    auto it = consumers.find(c);
    if (it == consumers.end() || it->second != 1) return false;
    if (!is_elementwise(parent[c]->operation)) return false;
    // The consumer's input slot must be the only owner (no array holds c).
    node *p = parent[c];
    for (uint8_t i = 0; i < p->num_inputs; i++)
      if (p->inputs[i].get() == c) return p->inputs[i].use_count() == 1;
    return false;
  };
  for (node *n : order) {
    if (n->evaluated) continue;
    if (attn_inner.count(n)) continue;  // computed inside a fused attention launch
    if (auto it = attention.find(n); it != attention.end()) {
      eval_attention(n, it->second);
      continue;
    }
    if (auto it = alias.find(n); it != alias.end()) {
      node *c = it->second;
      if (!c->evaluated) throw std::runtime_error("array: fused product not evaluated.");
      n->data = c->data;
      n->strides = c->strides;
      n->evaluated = true;
      continue;
    }
    if (auto it = relayout.find(n); it != relayout.end()) {
      // The product's output is this node's contiguous layout.
      node *c = it->second;
      if (!c->evaluated) throw std::runtime_error("array: relaid product not evaluated.");
      n->data = c->data;
      n->strides = contiguous_strides(n->shape);
      n->evaluated = true;
      continue;
    }
    if (!is_elementwise(n->operation)) {
      eval_node_nonfused(n);
    } else if (fusable(n)) {
      continue;  // computed by its consumer's program
    } else {
      // Collect the fused subtree below n.
      std::unordered_set<node *> fused{n};
      std::vector<node *> work{n};
      while (!work.empty()) {
        node *x = work.back();
        work.pop_back();
        for (uint8_t i = 0; i < x->num_inputs; i++) {
          node *c = x->inputs[i].get();
          if (fusable(c) && fused.insert(c).second) work.push_back(c);
        }
      }
      if (!try_program(n, fused)) {
        // Too large for one program: evaluate the subtree node by node.
        std::vector<node *> sub;
        for (node *m : order)
          if (fused.count(m) && m != n) sub.push_back(m);
        for (node *m : sub) {
          std::unordered_set<node *> one{m};
          if (!try_program(m, one)) throw std::runtime_error("array: elementwise node too large.");
        }
        std::unordered_set<node *> one{n};
        if (!try_program(n, one)) throw std::runtime_error("array: elementwise node too large.");
      }
    }
  }
  // Release inputs so intermediates are freed (include/array.h:2056-2060).
  for (node *n : order) {
    for (auto &i : n->inputs) i.reset();
    n->num_inputs = 0;
    n->residual.reset();
  }
}

}  // namespace detail

}  // namespace sil
