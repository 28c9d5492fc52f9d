// TEST INFRASTRUCTURE. CPU restatement of kurumi's reference interpreter for the ops of the
// kurumi_hip hot path. Each function cites the reference code it restates.
//
// Numeric contract (kurumi_core/src/dtype/traits/float.rs:8-72,105-161): f32/f64 compute
// natively; f16/bf16/f8 upcast to f32, compute, round back after EVERY primitive; integers
// wrap. Reductions fold sequentially left to right along the axis (interp/reduce.rs:67-84);
// sum/prod of low-precision floats accumulate in f32 and round once (reduce.rs:89-106).
#include <algorithm>
#include <cmath>
#include <cstring>
#include <functional>
#include <limits>
#include <stdexcept>

#include "oracle.h"

namespace kuo {

using ku::DType;
using ku::Node;
using ku::NodeId;
using ku::Op;
using ku::OpKind;
using ku::Shape;
using ku::Tensor;

namespace {

size_t numel(const Shape& s) { return ku::numel(s); }

bool is_lowp(DType d) { return d == DType::F16 || d == DType::BF16 || d == DType::F8E4M3 || d == DType::F8E5M2; }
bool is_fl(DType d) { return d == DType::F32 || is_lowp(d); }  // computed in f32

// element i of t as f64 (Elem::to_f64, dtype/traits/elem.rs:31-45)
double get_f64(const Tensor& t, size_t i) {
  const uint8_t* p = t.bytes.data() + i * ku::dt_width(t.dtype);
  switch (t.dtype) {
    case DType::BOOL: return *p ? 1.0 : 0.0;
    case DType::U8: return *p;
    case DType::U16: { uint16_t v; std::memcpy(&v, p, 2); return v; }
    case DType::U32: { uint32_t v; std::memcpy(&v, p, 4); return v; }
    case DType::U64: { uint64_t v; std::memcpy(&v, p, 8); return static_cast<double>(v); }
    case DType::I8: return static_cast<int8_t>(*p);
    case DType::I16: { int16_t v; std::memcpy(&v, p, 2); return v; }
    case DType::I32: { int32_t v; std::memcpy(&v, p, 4); return v; }
    case DType::I64: { int64_t v; std::memcpy(&v, p, 8); return static_cast<double>(v); }
    case DType::F8E4M3: return e4m3_to_f64(*p);
    case DType::F8E5M2: return e5m2_to_f64(*p);
    case DType::F16: { uint16_t v; std::memcpy(&v, p, 2); return f16_to_f64(v); }
    case DType::BF16: { uint16_t v; std::memcpy(&v, p, 2); return bf16_to_f32(v); }
    case DType::F32: { float v; std::memcpy(&v, p, 4); return v; }
    case DType::F64: { double v; std::memcpy(&v, p, 8); return v; }
    default: throw std::runtime_error("oracle: complex dtypes are out of scope");
  }
}

template <class I>
I sat(double x) {
  if (std::isnan(x)) return 0;
  if (x <= static_cast<double>(std::numeric_limits<I>::lowest())) return std::numeric_limits<I>::lowest();
  if (x >= static_cast<double>(std::numeric_limits<I>::max())) return std::numeric_limits<I>::max();
  return static_cast<I>(x);
}

// store f64 into element i with the target's from_f64 (elem.rs:31-45)
void put_f64(Tensor& t, size_t i, double x) {
  uint8_t* p = t.bytes.data() + i * ku::dt_width(t.dtype);
  switch (t.dtype) {
    case DType::BOOL: *p = (x != 0.0); break;
    case DType::U8: *p = sat<uint8_t>(x); break;
    case DType::U16: { uint16_t v = sat<uint16_t>(x); std::memcpy(p, &v, 2); } break;
    case DType::U32: { uint32_t v = sat<uint32_t>(x); std::memcpy(p, &v, 4); } break;
    case DType::U64: { uint64_t v = sat<uint64_t>(x); std::memcpy(p, &v, 8); } break;
    case DType::I8: { int8_t v = sat<int8_t>(x); std::memcpy(p, &v, 1); } break;
    case DType::I16: { int16_t v = sat<int16_t>(x); std::memcpy(p, &v, 2); } break;
    case DType::I32: { int32_t v = sat<int32_t>(x); std::memcpy(p, &v, 4); } break;
    case DType::I64: { int64_t v = sat<int64_t>(x); std::memcpy(p, &v, 8); } break;
    case DType::F8E4M3: *p = f32_to_e4m3(static_cast<float>(x)); break;
    case DType::F8E5M2: *p = f32_to_e5m2(static_cast<float>(x)); break;
    case DType::F16: { uint16_t v = f64_to_f16(x); std::memcpy(p, &v, 2); } break;
    case DType::BF16: { uint16_t v = f64_to_bf16(x); std::memcpy(p, &v, 2); } break;
    case DType::F32: { float v = static_cast<float>(x); std::memcpy(p, &v, 4); } break;
    case DType::F64: std::memcpy(p, &x, 8); break;
    default: throw std::runtime_error("oracle: complex dtypes are out of scope");
  }
}

Tensor make(DType dt, const Shape& s) {
  Tensor t;
  t.dtype = dt;
  t.shape = s;
  t.bytes.assign(numel(s) * ku::dt_width(dt), 0);
  return t;
}

// f32 view of a float-class tensor (exact for lowp)
std::vector<float> to_f32v(const Tensor& t) {
  size_t n = numel(t.shape);
  std::vector<float> v(n);
  if (t.dtype == DType::F32) {
    if (n) std::memcpy(v.data(), t.bytes.data(), n * 4);
  } else if (t.dtype == DType::BF16) {
    const uint16_t* p = reinterpret_cast<const uint16_t*>(t.bytes.data());
    for (size_t i = 0; i < n; ++i) v[i] = bf16_to_f32(p[i]);
  } else {
    for (size_t i = 0; i < n; ++i) v[i] = static_cast<float>(get_f64(t, i));
  }
  return v;
}
// round an f32 vector into dtype dt (from_f32 of float.rs)
Tensor from_f32v(DType dt, const Shape& s, const std::vector<float>& v) {
  Tensor t = make(dt, s);
  size_t n = v.size();
  if (dt == DType::F32) {
    if (n) std::memcpy(t.bytes.data(), v.data(), n * 4);
  } else if (dt == DType::BF16) {
    uint16_t* p = reinterpret_cast<uint16_t*>(t.bytes.data());
    for (size_t i = 0; i < n; ++i) p[i] = f32_to_bf16(v[i]);
  } else {
    for (size_t i = 0; i < n; ++i) put_f64(t, i, v[i]);
  }
  return t;
}

std::vector<double> to_f64v(const Tensor& t) {
  size_t n = numel(t.shape);
  std::vector<double> v(n);
  for (size_t i = 0; i < n; ++i) v[i] = get_f64(t, i);
  return v;
}

// integer elements as raw u64 bit patterns (sign-extended for signed types)
std::vector<uint64_t> to_u64v(const Tensor& t) {
  size_t n = numel(t.shape), w = ku::dt_width(t.dtype);
  std::vector<uint64_t> v(n);
  bool sgn = ku::dt_is_signed(t.dtype);
  for (size_t i = 0; i < n; ++i) {
    uint64_t x = 0;
    std::memcpy(&x, t.bytes.data() + i * w, w);
    if (sgn && w < 8 && (x >> (w * 8 - 1)) & 1) x |= ~0ull << (w * 8);
    v[i] = x;
  }
  return v;
}
Tensor from_u64v(DType dt, const Shape& s, const std::vector<uint64_t>& v) {
  Tensor t = make(dt, s);
  size_t w = ku::dt_width(dt);
  for (size_t i = 0; i < v.size(); ++i) std::memcpy(t.bytes.data() + i * w, &v[i], w);
  return t;
}
int64_t sext(uint64_t x, size_t w) {
  if (w == 8) return static_cast<int64_t>(x);
  uint64_t m = 1ull << (w * 8 - 1);
  x &= (m << 1) - 1;
  return static_cast<int64_t>((x ^ m) - m);
}
uint64_t trunc_w(uint64_t x, size_t w) { return w == 8 ? x : (x & ((1ull << (w * 8)) - 1)); }

// ---------------- elementwise (interp/elementwise.rs:7-100) ----------------

Tensor elementwise(const Op& op, DType out_dt, const std::vector<const Tensor*>& in) {
  const Tensor& a = *in[0];
  const Shape& s = a.shape;
  size_t n = numel(s);
  DType dt = a.dtype;
  switch (op.kind) {
    case OpKind::Cast: {  // dtype/convert.rs:14-47 (through f64)
      Tensor o = make(op.to, s);
      if (dt == op.to) return a;
      for (size_t i = 0; i < n; ++i) put_f64(o, i, get_f64(a, i));
      return o;
    }
    case OpKind::Bitcast: {  // convert.rs:150-152
      Tensor o = a;
      o.dtype = op.to;
      if (op.to == DType::BOOL)
        for (auto& b : o.bytes) b = b != 0;
      return o;
    }
    case OpKind::CmpLt: case OpKind::CmpEq: {
      Tensor o = make(DType::BOOL, s);
      const Tensor& b = *in[1];
      bool lt = op.kind == OpKind::CmpLt;
      if (ku::dt_is_int(dt)) {
        auto x = to_u64v(a), y = to_u64v(b);
        bool sg = ku::dt_is_signed(dt);
        for (size_t i = 0; i < n; ++i)
          o.bytes[i] = lt ? (sg ? (int64_t)x[i] < (int64_t)y[i] : x[i] < y[i]) : x[i] == y[i];
      } else if (dt == DType::BOOL) {
        for (size_t i = 0; i < n; ++i) o.bytes[i] = lt ? (a.bytes[i] < b.bytes[i]) : (a.bytes[i] == b.bytes[i]);
      } else {
        for (size_t i = 0; i < n; ++i) {
          double x = get_f64(a, i), y = get_f64(b, i);
          o.bytes[i] = lt ? (x < y) : (x == y);
        }
      }
      return o;
    }
    case OpKind::Where: {  // select_k
      const Tensor &x = *in[1], &y = *in[2];
      Tensor o = make(x.dtype, s);
      size_t w = ku::dt_width(x.dtype);
      for (size_t i = 0; i < n; ++i)
        std::memcpy(o.bytes.data() + i * w, (a.bytes[i] ? x : y).bytes.data() + i * w, w);
      return o;
    }
    default: break;
  }
  if (dt == DType::BOOL) {  // bitwise on bool
    const Tensor& b = *in[1];
    Tensor o = make(DType::BOOL, s);
    for (size_t i = 0; i < n; ++i) {
      bool x = a.bytes[i], y = b.bytes[i];
      o.bytes[i] = op.kind == OpKind::And ? (x && y) : op.kind == OpKind::Or ? (x || y) : (x != y);
    }
    return o;
  }
  if (ku::dt_is_int(dt)) {
    size_t w = ku::dt_width(dt);
    bool sg = ku::dt_is_signed(dt);
    auto x = to_u64v(a);
    std::vector<uint64_t> y;
    if (in.size() > 1) y = to_u64v(*in[1]);
    std::vector<uint64_t> r(n);
    for (size_t i = 0; i < n; ++i) {
      uint64_t u = x[i], v = y.empty() ? 0 : y[i];
      uint64_t out;
      switch (op.kind) {
        case OpKind::Add: out = u + v; break;
        case OpKind::Mul: out = u * v; break;
        case OpKind::Max: out = sg ? ((int64_t)u >= (int64_t)v ? u : v) : (u >= v ? u : v); break;
        case OpKind::Neg: out = 0 - u; break;
        case OpKind::IDiv:
          if (trunc_w(v, w) == 0) out = 0;
          else if (sg) {
            int64_t p = sext(u, w), q = sext(v, w);
            out = (q == -1) ? (uint64_t)(0 - (uint64_t)p) : (uint64_t)(p / q);
          } else {
            out = trunc_w(u, w) / trunc_w(v, w);
          }
          break;
        case OpKind::And: out = u & v; break;
        case OpKind::Or: out = u | v; break;
        case OpKind::Xor: out = u ^ v; break;
        case OpKind::Shl: out = trunc_w(u, w) << (v & (w * 8 - 1)); break;
        case OpKind::Shr:
          out = sg ? (uint64_t)(sext(u, w) >> (v & (w * 8 - 1))) : (trunc_w(u, w) >> (v & (w * 8 - 1)));
          break;
        default: throw std::runtime_error(std::string("oracle: int op ") + ku::op_name(op.kind));
      }
      r[i] = trunc_w(out, w);
    }
    return from_u64v(dt, s, r);
  }
  if (dt == DType::F64) {
    auto x = to_f64v(a);
    std::vector<double> y;
    if (in.size() > 1) y = to_f64v(*in[1]);
    Tensor o = make(dt, s);
    double* r = reinterpret_cast<double*>(o.bytes.data());
    for (size_t i = 0; i < n; ++i) {
      double u = x[i];
      switch (op.kind) {
        case OpKind::Add: r[i] = u + y[i]; break;
        case OpKind::Mul: r[i] = u * y[i]; break;
        case OpKind::Max: r[i] = std::fmax(u, y[i]); break;
        case OpKind::Neg: r[i] = -u; break;
        case OpKind::Recip: r[i] = 1.0 / u; break;
        case OpKind::Sqrt: r[i] = std::sqrt(u); break;
        case OpKind::Exp2: r[i] = std::exp2(u); break;
        case OpKind::Log2: r[i] = std::log2(u); break;
        case OpKind::Sin: r[i] = std::sin(u); break;
        case OpKind::Floor: r[i] = std::floor(u); break;
        default: throw std::runtime_error(std::string("oracle: f64 op ") + ku::op_name(op.kind));
      }
    }
    return o;
  }
  // f32 and low-precision floats: compute in f32, round to the dtype (float.rs)
  std::vector<float> x = to_f32v(a), y;
  if (in.size() > 1) y = to_f32v(*in[1]);
  std::vector<float> r(n);
  switch (op.kind) {
    case OpKind::Add: for (size_t i = 0; i < n; ++i) r[i] = x[i] + y[i]; break;
    case OpKind::Mul: for (size_t i = 0; i < n; ++i) r[i] = x[i] * y[i]; break;
    case OpKind::Max: for (size_t i = 0; i < n; ++i) r[i] = std::fmax(x[i], y[i]); break;
    case OpKind::Neg: for (size_t i = 0; i < n; ++i) r[i] = -x[i]; break;
    case OpKind::Recip: for (size_t i = 0; i < n; ++i) r[i] = 1.0f / x[i]; break;
    case OpKind::Sqrt: for (size_t i = 0; i < n; ++i) r[i] = std::sqrt(x[i]); break;
    case OpKind::Exp2: for (size_t i = 0; i < n; ++i) r[i] = exp2f(x[i]); break;
    case OpKind::Log2: for (size_t i = 0; i < n; ++i) r[i] = log2f(x[i]); break;
    case OpKind::Sin: for (size_t i = 0; i < n; ++i) r[i] = sinf(x[i]); break;
    case OpKind::Floor: for (size_t i = 0; i < n; ++i) r[i] = floorf(x[i]); break;
    default: throw std::runtime_error(std::string("oracle: float op ") + ku::op_name(op.kind));
  }
  (void)out_dt;
  return from_f32v(dt, s, r);
}

// ---------------- movement (interp/movement.rs:7-160) ----------------

void inc(std::vector<size_t>& c, const Shape& s) {
  for (size_t i = c.size(); i-- > 0;) {
    if (++c[i] < s[i]) return;
    c[i] = 0;
  }
}

Tensor movement(const Op& op, const Tensor& a, const Shape& out_shape) {
  if (op.kind == OpKind::Reshape) {
    Tensor o = a;
    o.shape = op.shape;
    return o;
  }
  size_t w = ku::dt_width(a.dtype);
  Tensor o = make(a.dtype, out_shape);
  auto st = ku::row_major_strides(a.shape);
  std::vector<size_t> c(out_shape.size(), 0);
  size_t n = numel(out_shape);
  for (size_t f = 0; f < n; ++f) {
    bool zero = false;
    size_t src = 0;
    for (size_t d = 0; d < out_shape.size(); ++d) {
      switch (op.kind) {
        case OpKind::Expand: src += a.shape[d] == 1 ? 0 : c[d] * st[d]; break;
        case OpKind::Permute: src += c[d] * st[op.perm[d]]; break;
        case OpKind::Slice: src += (op.ranges[d].start + c[d] * op.ranges[d].step) * st[d]; break;
        case OpKind::Flip: {
          bool fl = std::find(op.axes.begin(), op.axes.end(), d) != op.axes.end();
          src += (fl ? a.shape[d] - 1 - c[d] : c[d]) * st[d];
        } break;
        case OpKind::Pad: {
          int64_t sc = static_cast<int64_t>(c[d]) - static_cast<int64_t>(op.pads[d].lo);
          if (sc < 0 || sc >= static_cast<int64_t>(a.shape[d])) zero = true;
          else src += static_cast<size_t>(sc) * st[d];
        } break;
        default: throw std::runtime_error("oracle: not a movement op");
      }
    }
    if (!zero) std::memcpy(o.bytes.data() + f * w, a.bytes.data() + src * w, w);
    inc(c, out_shape);
  }
  return o;
}

// ---------------- reductions (interp/reduce.rs:18-106) ----------------

struct AxisIter {
  size_t outer, len, inner;
};
AxisIter axis_iter(const Shape& s, size_t axis) {
  AxisIter it{1, s[axis], 1};
  for (size_t d = 0; d < axis; ++d) it.outer *= s[d];
  for (size_t d = axis + 1; d < s.size(); ++d) it.inner *= s[d];
  return it;
}

Tensor reduce(const Op& op, const Tensor& a) {
  size_t axis = op.axis;
  Shape os = a.shape;
  os.erase(os.begin() + axis);
  AxisIter it = axis_iter(a.shape, axis);
  DType dt = a.dtype;
  if (op.kind == OpKind::ArgReduce) {  // arg_reduce_t: strict compare, first index wins
    // interp/reduce.rs:46 reads element 0 of the axis before the loop: an empty axis with a
    // non-empty output is out of bounds there (a panic); here an error
    if (it.len == 0 && it.outer * it.inner > 0) throw std::runtime_error("arg_reduce over an empty axis");
    Tensor o = make(DType::I64, os);
    int64_t* r = reinterpret_cast<int64_t*>(o.bytes.data());
    bool mn = op.arg == ku::ArgKind::Min;
    if (ku::dt_is_int(dt)) {
      auto v = to_u64v(a);
      bool sg = ku::dt_is_signed(dt);
      auto gt = [&](uint64_t x, uint64_t y) { return sg ? (int64_t)x > (int64_t)y : x > y; };
      for (size_t p = 0; p < it.outer; ++p)
        for (size_t q = 0; q < it.inner; ++q) {
          size_t base = p * it.len * it.inner + q;
          uint64_t best = v[base];
          int64_t bi = 0;
          for (size_t k = 1; k < it.len; ++k) {
            uint64_t x = v[base + k * it.inner];
            if (mn ? gt(best, x) : gt(x, best)) { best = x; bi = (int64_t)k; }
          }
          r[p * it.inner + q] = bi;
        }
    } else {
      std::vector<double> v = (dt == DType::F64) ? to_f64v(a) : std::vector<double>();
      std::vector<float> vf = (dt != DType::F64) ? to_f32v(a) : std::vector<float>();
      for (size_t p = 0; p < it.outer; ++p)
        for (size_t q = 0; q < it.inner; ++q) {
          size_t base = p * it.len * it.inner + q;
          auto at = [&](size_t k) { return dt == DType::F64 ? v[base + k * it.inner] : (double)vf[base + k * it.inner]; };
          double best = at(0);
          int64_t bi = 0;
          for (size_t k = 1; k < it.len; ++k) {
            double x = at(k);
            if (mn ? (x < best) : (x > best)) { best = x; bi = (int64_t)k; }
          }
          r[p * it.inner + q] = bi;
        }
    }
    return o;
  }
  bool is_sum = op.kind == OpKind::Sum, is_prod = op.kind == OpKind::Prod;
  if (ku::dt_is_int(dt)) {
    auto v = to_u64v(a);
    bool sg = ku::dt_is_signed(dt);
    size_t w = ku::dt_width(dt);
    std::vector<uint64_t> r(it.outer * it.inner);
    for (size_t p = 0; p < it.outer; ++p)
      for (size_t q = 0; q < it.inner; ++q) {
        size_t base = p * it.len * it.inner + q;
        uint64_t acc;
        if (is_sum) acc = 0;
        else if (is_prod) acc = 1;
        else acc = sg ? (uint64_t)(-(int64_t)(1ull << (w * 8 - 1))) : 0;  // MIN
        if (!is_sum && !is_prod && sg && w == 8) acc = (uint64_t)std::numeric_limits<int64_t>::min();
        for (size_t k = 0; k < it.len; ++k) {
          uint64_t x = v[base + k * it.inner];
          if (is_sum) acc += x;
          else if (is_prod) acc *= x;
          else acc = sg ? ((int64_t)x > (int64_t)acc ? x : acc) : (x > acc ? x : acc);
        }
        r[p * it.inner + q] = trunc_w(acc, w);
      }
    return from_u64v(dt, os, r);
  }
  if (dt == DType::F64) {
    auto v = to_f64v(a);
    Tensor o = make(dt, os);
    double* r = reinterpret_cast<double*>(o.bytes.data());
    for (size_t p = 0; p < it.outer; ++p)
      for (size_t q = 0; q < it.inner; ++q) {
        size_t base = p * it.len * it.inner + q;
        double acc = is_sum ? 0.0 : is_prod ? 1.0 : -INFINITY;
        for (size_t k = 0; k < it.len; ++k) {
          double x = v[base + k * it.inner];
          acc = is_sum ? acc + x : is_prod ? acc * x : std::fmax(acc, x);
        }
        r[p * it.inner + q] = acc;
      }
    return o;
  }
  // f32 / lowp: promoted f32 accumulation (sum/prod) or max in f32 (exact for lowp)
  auto v = to_f32v(a);
  std::vector<float> r(it.outer * it.inner);
  float init = is_sum ? 0.f : is_prod ? 1.f : -INFINITY;
  if (!is_sum && !is_prod && dt == DType::F8E4M3) init = -448.f;  // F8E4M3::from_f32(f32::MIN) saturates
  for (size_t p = 0; p < it.outer; ++p) {
    if (it.inner == 1) {
      const float* row = v.data() + p * it.len;
      float acc = init;
      if (is_sum) for (size_t k = 0; k < it.len; ++k) acc = acc + row[k];
      else if (is_prod) for (size_t k = 0; k < it.len; ++k) acc = acc * row[k];
      else for (size_t k = 0; k < it.len; ++k) acc = std::fmax(acc, row[k]);
      r[p] = acc;
      continue;
    }
    for (size_t q = 0; q < it.inner; ++q) {
      size_t base = p * it.len * it.inner + q;
      float acc = init;
      for (size_t k = 0; k < it.len; ++k) {
        float x = v[base + k * it.inner];
        acc = is_sum ? acc + x : is_prod ? acc * x : std::fmax(acc, x);
      }
      r[p * it.inner + q] = acc;
    }
  }
  return from_f32v(dt, os, r);
}

// ---------------- nn (interp/nn.rs:18-172) ----------------

template <class T>
void softmax_lines(std::vector<T>& d, const Shape& s, size_t axis, bool rms, T eps) {
  AxisIter it = axis_iter(s, axis);
  for (size_t p = 0; p < it.outer; ++p)
    for (size_t q = 0; q < it.inner; ++q) {
      size_t base = p * it.len * it.inner + q;
      if (!rms) {
        T m = -std::numeric_limits<T>::infinity();
        for (size_t k = 0; k < it.len; ++k) m = std::fmax(m, d[base + k * it.inner]);
        T sum = 0;
        for (size_t k = 0; k < it.len; ++k) {
          T e = std::exp(d[base + k * it.inner] - m);
          d[base + k * it.inner] = e;
          sum += e;
        }
        for (size_t k = 0; k < it.len; ++k) d[base + k * it.inner] /= sum;
      } else {
        T ss = 0;
        for (size_t k = 0; k < it.len; ++k) {
          T x = d[base + k * it.inner];
          ss += x * x;
        }
        T r = std::sqrt(ss / static_cast<T>(it.len) + eps);
        for (size_t k = 0; k < it.len; ++k) d[base + k * it.inner] /= r;
      }
    }
}

Tensor rowop(const Op& op, const Tensor& a) {
  bool rms = op.kind == OpKind::RmsNorm;
  if (a.dtype == DType::F64) {
    auto v = to_f64v(a);
    softmax_lines<double>(v, a.shape, op.axis, rms, static_cast<double>(op.eps));
    Tensor o = make(DType::F64, a.shape);
    std::memcpy(o.bytes.data(), v.data(), v.size() * 8);
    return o;
  }
  auto v = to_f32v(a);
  softmax_lines<float>(v, a.shape, op.axis, rms, op.eps);
  return from_f32v(a.dtype, a.shape, v);
}

// dot_general (interp/contract.rs:26-166): out = batch ++ lhs_free ++ rhs_free; f32 and
// promoted low-precision accumulate sequentially over the contraction in f32, f64 in f64,
// ints wrap; low-precision results round once to the input dtype.
std::vector<size_t> offsets(const Shape& s, const std::vector<size_t>& st, const std::vector<size_t>& axes) {
  Shape sub;
  for (size_t a : axes) sub.push_back(s[a]);
  size_t n = numel(sub);
  std::vector<size_t> off(n);
  std::vector<size_t> c(sub.size(), 0);
  for (size_t i = 0; i < n; ++i) {
    size_t o = 0;
    for (size_t j = 0; j < axes.size(); ++j) o += c[j] * st[axes[j]];
    off[i] = o;
    inc(c, sub);
  }
  return off;
}

Tensor dot(const Op& op, const Tensor& a, const Tensor& b, const Shape& out_shape) {
  auto sa = ku::row_major_strides(a.shape), sb = ku::row_major_strides(b.shape);
  auto af = ku::free_axes(a.shape.size(), op.lb, op.lc), bf = ku::free_axes(b.shape.size(), op.rb, op.rc);
  auto ab_off = offsets(a.shape, sa, op.lb), bb_off = offsets(b.shape, sb, op.rb);
  auto af_off = offsets(a.shape, sa, af), bf_off = offsets(b.shape, sb, bf);
  auto ac_off = offsets(a.shape, sa, op.lc), bc_off = offsets(b.shape, sb, op.rc);
  size_t NB = ab_off.size(), M = af_off.size(), N = bf_off.size(), K = ac_off.size();
  DType dt = a.dtype;
  if (ku::dt_is_int(dt)) {
    auto x = to_u64v(a), y = to_u64v(b);
    std::vector<uint64_t> r(NB * M * N);
    for (size_t bi = 0; bi < NB; ++bi)
      for (size_t i = 0; i < M; ++i)
        for (size_t j = 0; j < N; ++j) {
          uint64_t acc = 0;
          for (size_t k = 0; k < K; ++k)
            acc += x[ab_off[bi] + af_off[i] + ac_off[k]] * y[bb_off[bi] + bf_off[j] + bc_off[k]];
          r[(bi * M + i) * N + j] = trunc_w(acc, ku::dt_width(dt));
        }
    return from_u64v(dt, out_shape, r);
  }
  if (dt == DType::F64) {
    auto x = to_f64v(a), y = to_f64v(b);
    Tensor o = make(dt, out_shape);
    double* r = reinterpret_cast<double*>(o.bytes.data());
    for (size_t bi = 0; bi < NB; ++bi)
      for (size_t i = 0; i < M; ++i)
        for (size_t j = 0; j < N; ++j) {
          double acc = 0;
          for (size_t k = 0; k < K; ++k) acc += x[ab_off[bi] + af_off[i] + ac_off[k]] * y[bb_off[bi] + bf_off[j] + bc_off[k]];
          r[(bi * M + i) * N + j] = acc;
        }
    return o;
  }
  std::vector<float> x = to_f32v(a), y = to_f32v(b);
  std::vector<float> r(NB * M * N);
  // gather the rhs so the inner loop streams contiguous memory
  std::vector<float> yt(K * N);
  std::vector<float> xr(K);
  for (size_t bi = 0; bi < NB; ++bi) {
    for (size_t j = 0; j < N; ++j)
      for (size_t k = 0; k < K; ++k) yt[j * K + k] = y[bb_off[bi] + bf_off[j] + bc_off[k]];
    for (size_t i = 0; i < M; ++i) {
      for (size_t k = 0; k < K; ++k) xr[k] = x[ab_off[bi] + af_off[i] + ac_off[k]];
      float* out = r.data() + (bi * M + i) * N;
      for (size_t j = 0; j < N; ++j) {
        const float* yy = yt.data() + j * K;
        float acc = 0.f;
        for (size_t k = 0; k < K; ++k) acc = acc + xr[k] * yy[k];
        out[j] = acc;
      }
    }
  }
  return from_f32v(dt, out_shape, r);
}

// quant_matmul (interp/contract.rs:69-99): dequantize the packed weight exactly as
// quant.rs:100-133 does (raw field, low field first; asymmetric q*s + min, symmetric
// sign-extended q*s, f16 scale/min widened to f32), then act (cast to f32) x W^T through the
// f32 contraction above, and the result cast back to act's dtype.
Tensor quant_matmul(const Op& op, const Tensor& act, const Tensor& qw, const Tensor& scales, const Tensor* mins,
                    const Shape& out_shape) {
  const size_t m = act.shape[0], k = act.shape[1], n = qw.shape[0];
  const int bits = op.qbits;
  const size_t g = op.qgroup, ng = k / g, rb = k * bits / 8, per = 8 / bits;
  const uint8_t* pk = qw.bytes.data();
  auto f16 = [](const Tensor& t, size_t i) {
    uint16_t h;
    std::memcpy(&h, t.bytes.data() + 2 * i, 2);
    return static_cast<float>(f16_to_f64(h));
  };
  Tensor w = make(DType::F32, {n, k});
  float* wp = reinterpret_cast<float*>(w.bytes.data());
  for (size_t r = 0; r < n; ++r)
    for (size_t c = 0; c < k; ++c) {
      const uint32_t raw = (pk[r * rb + c / per] >> ((c % per) * bits)) & ((1u << bits) - 1);
      const size_t gi = r * ng + c / g;
      const float s = f16(scales, gi);
      float v;
      if (mins) {
        v = static_cast<float>(raw) * s + f16(*mins, gi);
      } else {
        const int sh = 32 - bits;
        v = static_cast<float>(static_cast<int32_t>(raw << sh) >> sh) * s;
      }
      wp[r * k + c] = v;
    }
  Tensor af = make(DType::F32, {m, k});
  {
    auto x = to_f32v(act);
    std::memcpy(af.bytes.data(), x.data(), x.size() * 4);
  }
  Op d;
  d.kind = OpKind::DotGeneral;
  d.lc = {1};
  d.rc = {1};
  Tensor r = dot(d, af, w, out_shape);
  return from_f32v(act.dtype, out_shape, to_f32v(r));
}

// scale_causal (interp/nn.rs:154-172)
Tensor scale_causal(const Tensor& raw, float scale, size_t s, bool causal) {
  if (raw.dtype == DType::F64) {
    auto v = to_f64v(raw);
    for (size_t base = 0; base < v.size(); base += s * s)
      for (size_t i = 0; i < s; ++i)
        for (size_t j = 0; j < s; ++j) {
          double& e = v[base + i * s + j];
          e = (causal && j > i) ? -INFINITY : e * static_cast<double>(scale);
        }
    Tensor o = make(DType::F64, raw.shape);
    std::memcpy(o.bytes.data(), v.data(), v.size() * 8);
    return o;
  }
  auto v = to_f32v(raw);
  for (size_t base = 0; base < v.size(); base += s * s)
    for (size_t i = 0; i < s; ++i)
      for (size_t j = 0; j < s; ++j) {
        float& e = v[base + i * s + j];
        e = (causal && j > i) ? -INFINITY : e * scale;
      }
  return from_f32v(raw.dtype, raw.shape, v);
}

Tensor sdpa(const Tensor& q, const Tensor& k, const Tensor& v, bool causal) {
  size_t r = q.shape.size();
  size_t s = q.shape[r - 2], dh = q.shape[r - 1];
  std::vector<size_t> batch;
  for (size_t i = 0; i + 2 < r; ++i) batch.push_back(i);
  Op d1;
  d1.kind = OpKind::DotGeneral;
  d1.lc = {r - 1};
  d1.rc = {r - 1};
  d1.lb = batch;
  d1.rb = batch;
  Shape rs(q.shape.begin(), q.shape.end() - 1);
  rs.push_back(s);
  Tensor raw = dot(d1, q, k, rs);
  Tensor sc = scale_causal(raw, 1.0f / std::sqrt(static_cast<float>(dh)), s, causal);
  Op sm;
  sm.kind = OpKind::Softmax;
  sm.axis = r - 1;
  Tensor attn = rowop(sm, sc);
  Op d2 = d1;
  d2.rc = {r - 2};
  return dot(d2, attn, v, q.shape);
}

Tensor eval_op(const Node& n, const std::vector<const Tensor*>& in) {
  const Op& op = n.op;
  switch (op.kind) {
    case OpKind::Const: {
      Tensor t;
      t.dtype = op.data_dtype;
      t.shape = op.shape;
      t.bytes.assign(op.data->begin(), op.data->end());
      return t;
    }
    case OpKind::Detach: return *in[0];
    case OpKind::Iota: {  // convert.rs:76-82
      Tensor t = make(op.to, op.shape);
      size_t stride = 1;
      for (size_t d = op.axis + 1; d < op.shape.size(); ++d) stride *= op.shape[d];
      for (size_t f = 0; f < numel(op.shape); ++f) put_f64(t, f, static_cast<double>((f / stride) % op.shape[op.axis]));
      return t;
    }
    case OpKind::RandUniform: {  // interp/random.rs:24-28
      uint64_t seed = static_cast<uint64_t>(static_cast<int64_t>(get_f64(*in[0], 0)));
      if (ku::dt_is_int(in[0]->dtype)) seed = static_cast<uint64_t>(sext(to_u64v(*in[0])[0], ku::dt_width(in[0]->dtype)));
      Tensor t = make(DType::F32, op.shape);
      float* p = reinterpret_cast<float*>(t.bytes.data());
      for (size_t i = 0; i < numel(op.shape); ++i) p[i] = uniform_f32(threefry2x32(seed, i));
      return t;
    }
    case OpKind::Sum: case OpKind::Prod: case OpKind::ReduceMax: case OpKind::ArgReduce: return reduce(op, *in[0]);
    case OpKind::Softmax: case OpKind::RmsNorm: return rowop(op, *in[0]);
    case OpKind::Sdpa: return sdpa(*in[0], *in[1], *in[2], op.causal);
    case OpKind::Reshape: case OpKind::Expand: case OpKind::Permute: case OpKind::Slice: case OpKind::Flip:
    case OpKind::Pad:
      return movement(op, *in[0], n.shape);
    case OpKind::DotGeneral: return dot(op, *in[0], *in[1], n.shape);
    case OpKind::QuantMatmul: return quant_matmul(op, *in[0], *in[1], *in[2], in.size() > 3 ? in[3] : nullptr, n.shape);
    case OpKind::Input: throw std::runtime_error("oracle: Input must come from feeds");
    default: return elementwise(op, n.dtype, in);
  }
}

}  // namespace

Tensor cast(const Tensor& t, DType to) {
  Op op;
  op.kind = OpKind::Cast;
  op.to = to;
  return elementwise(op, to, {&t});
}

// interp.rs:42-60: memoised walk; shared subgraphs compute once. Buffers are dropped after
// their last consumer to bound peak memory.
std::vector<Tensor> interpret(const ku::Graph& g, const std::vector<NodeId>& roots, const ku::Feeds& feeds) {
  auto order = ku::reachable_multi(g, roots);
  std::sort(order.begin(), order.end());
  std::vector<int> uses(g.size(), 0);
  for (NodeId id : order)
    for (NodeId s : g.node(id).src) uses[s]++;
  for (NodeId r : roots) uses[r]++;
  std::vector<std::shared_ptr<Tensor>> memo(g.size());
  for (NodeId id : order) {
    const Node& n = g.node(id);
    if (n.op.kind == OpKind::Input) {
      auto it = feeds.find(id);
      if (it == feeds.end()) throw std::runtime_error("interpret: missing feed for an Input node");
      memo[id] = std::make_shared<Tensor>(*it->second);
      continue;
    }
    std::vector<const Tensor*> in;
    for (NodeId s : n.src) in.push_back(memo[s].get());
    memo[id] = std::make_shared<Tensor>(eval_op(n, in));
    for (NodeId s : n.src)
      if (--uses[s] == 0) memo[s].reset();
  }
  std::vector<Tensor> out;
  for (NodeId r : roots) out.push_back(*memo[r]);
  return out;
}

}  // namespace kuo
