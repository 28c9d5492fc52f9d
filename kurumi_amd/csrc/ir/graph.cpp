// IR arena, inference, record-time checks and builders. See graph.h for the reference map.
#include "graph.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <sstream>
#include <unordered_set>

namespace ku {

static std::atomic<uint64_t> g_graph_counter{1};

const char* op_name(OpKind k) {
  static const char* n[] = {"Const", "Input", "Iota", "RandUniform", "Cast", "Bitcast", "Detach",
                            "Add", "Mul", "Max", "Neg", "IDiv", "And", "Or", "Xor", "Shl", "Shr",
                            "CmpLt", "CmpEq", "Where", "Recip", "Sqrt", "Exp2", "Log2", "Sin", "Floor",
                            "Sum", "Prod", "ReduceMax", "ArgReduce", "Softmax", "RmsNorm", "Sdpa",
                            "Reshape", "Permute", "Expand", "Slice", "Flip", "Pad", "DotGeneral",
                            "QuantMatmul"};
  uint32_t i = static_cast<uint32_t>(k);
  return i < static_cast<uint32_t>(OpKind::NumKinds) ? n[i] : "?";
}

std::vector<size_t> row_major_strides(const Shape& s) {
  std::vector<size_t> st(s.size(), 1);
  for (size_t i = s.size(); i-- > 1;) st[i - 1] = st[i] * s[i];
  return st;
}

std::vector<size_t> free_axes(size_t rank, const std::vector<size_t>& batch, const std::vector<size_t>& contract) {
  std::vector<size_t> out;
  for (size_t i = 0; i < rank; ++i)
    if (std::find(batch.begin(), batch.end(), i) == batch.end() &&
        std::find(contract.begin(), contract.end(), i) == contract.end())
      out.push_back(i);
  return out;
}

std::string shape_str(const Shape& s) {
  std::ostringstream o;
  o << "[";
  for (size_t i = 0; i < s.size(); ++i) o << (i ? ", " : "") << s[i];
  o << "]";
  return o.str();
}

Graph::Graph() : id_(g_graph_counter.fetch_add(1)) {}

const Node& Graph::node(NodeId i) const {
  if (i >= nodes_.size()) throw Error("node id " + std::to_string(i) + " out of range");
  return nodes_[i];
}

void Graph::check_id(const char* op, NodeId a) const {
  if (a >= nodes_.size()) throw Error(std::string(op) + ": node id " + std::to_string(a) + " out of range");
}

void Graph::same_shape(const char* op, NodeId a, NodeId b) const {
  if (shape(a) != shape(b)) throw Error(std::string(op) + ": " + shape_str(shape(a)) + " vs " + shape_str(shape(b)));
}
void Graph::same_dtype(const char* op, NodeId a, NodeId b) const {
  if (dtype(a) != dtype(b))
    throw Error(std::string(op) + ": dtype " + dt_name(dtype(a)) + " vs " + dt_name(dtype(b)));
}
void Graph::require(const char* op, NodeId a, bool ok, const char* want) const {
  if (!ok) throw Error(std::string(op) + ": " + want + " dtype required, got " + dt_name(dtype(a)));
}
void Graph::reduce_axis_ok(const char* op, NodeId a, size_t axis) const {
  size_t r = shape(a).size();
  if (axis >= r)
    throw Error(std::string(op) + ": axis " + std::to_string(axis) + " out of range for rank " + std::to_string(r));
}

// graph/infer.rs:12-38
DType Graph::infer_dtype(const Op& op, const std::vector<NodeId>& src) const {
  switch (op.kind) {
    case OpKind::Const: return op.data_dtype;
    case OpKind::Input: case OpKind::Iota: return op.to;
    case OpKind::Cast: case OpKind::Bitcast: return op.to;
    case OpKind::CmpLt: case OpKind::CmpEq: return DType::BOOL;
    case OpKind::ArgReduce: return DType::I64;
    case OpKind::RandUniform: return DType::F32;
    case OpKind::Where: return dtype(src[1]);
    default: return dtype(src[0]);
  }
}

// graph/infer.rs:42-134 (subset that this IR records)
Shape Graph::derive_shape(const Op& op, const std::vector<NodeId>& src) const {
  auto is = [&](size_t i) -> const Shape& { return shape(src[i]); };
  switch (op.kind) {
    case OpKind::Const: case OpKind::Input: case OpKind::Iota: case OpKind::RandUniform: return op.shape;
    case OpKind::Sum: case OpKind::Prod: case OpKind::ReduceMax: case OpKind::ArgReduce: {
      Shape s = is(0);
      s.erase(s.begin() + op.axis);
      return s;
    }
    case OpKind::Reshape: case OpKind::Expand: return op.shape;
    case OpKind::Permute: {
      Shape s;
      for (size_t p : op.perm) s.push_back(is(0)[p]);
      return s;
    }
    case OpKind::Slice: {
      Shape s;
      for (auto& r : op.ranges) s.push_back((r.end - r.start + r.step - 1) / r.step);
      return s;
    }
    case OpKind::Pad: {
      Shape s;
      for (size_t i = 0; i < op.pads.size(); ++i) s.push_back(op.pads[i].lo + is(0)[i] + op.pads[i].hi);
      return s;
    }
    case OpKind::DotGeneral: {
      const Shape &a = is(0), &b = is(1);
      Shape s;
      for (size_t i : op.lb) s.push_back(a[i]);
      for (size_t i : free_axes(a.size(), op.lb, op.lc)) s.push_back(a[i]);
      for (size_t i : free_axes(b.size(), op.rb, op.rc)) s.push_back(b[i]);
      return s;
    }
    case OpKind::QuantMatmul: return {is(0)[0], is(1)[0]};  // infer.rs:132
    default: return is(0);  // elementwise, Softmax, RmsNorm, Sdpa, Flip
  }
}

NodeId Graph::push(Op op, std::vector<NodeId> src) {
  for (NodeId s : src) check_id(op_name(op.kind), s);
  Node n;
  n.dtype = infer_dtype(op, src);
  n.shape = derive_shape(op, src);
  n.op = std::move(op);
  n.src = std::move(src);
  nodes_.push_back(std::move(n));
  return static_cast<NodeId>(nodes_.size() - 1);
}

// ---------------- leaves ----------------

NodeId Graph::constant_bytes(DType dt, const uint8_t* bytes, size_t nbytes, const Shape& shape) {
  size_t want = numel(shape) * dt_width(dt);
  if (nbytes != want)
    throw Error("constant: " + std::to_string(nbytes) + " bytes for " + std::to_string(numel(shape)) + " x " +
                dt_name(dt));
  Op op;
  op.kind = OpKind::Const;
  op.shape = shape;
  op.data_dtype = dt;
  op.data = std::make_shared<const std::vector<uint8_t>>(bytes, bytes + nbytes);
  return push(std::move(op), {});
}

NodeId Graph::constant_f32(const std::vector<float>& v, const Shape& shape) {
  return constant_bytes(DType::F32, reinterpret_cast<const uint8_t*>(v.data()), v.size() * 4, shape);
}

NodeId Graph::input(const Shape& shape, DType dt) {
  Op op;
  op.kind = OpKind::Input;
  op.shape = shape;
  op.to = dt;
  return push(std::move(op), {});
}

NodeId Graph::iota(const Shape& shape, size_t axis, DType dt) {
  if (axis >= shape.size()) throw Error("iota: axis out of range");
  Op op;
  op.kind = OpKind::Iota;
  op.shape = shape;
  op.axis = axis;
  op.to = dt;
  return push(std::move(op), {});
}

// random.rs:11-14: the seed is an I64 const [1] feeding RandUniform.
NodeId Graph::rand_uniform(const Shape& shape, uint64_t seed) {
  int64_t s = static_cast<int64_t>(seed);
  NodeId sn = constant_bytes(DType::I64, reinterpret_cast<const uint8_t*>(&s), 8, {1});
  return rand_uniform_seeded(shape, sn);
}
NodeId Graph::rand_uniform_seeded(const Shape& shape, NodeId seed) {
  check_id("rand_uniform", seed);
  if (numel(this->shape(seed)) != 1) throw Error("rand_uniform: seed must hold one element");
  Op op;
  op.kind = OpKind::RandUniform;
  op.shape = shape;
  return push(std::move(op), {seed});
}

NodeId Graph::cast(NodeId a, DType to) {
  Op op;
  op.kind = OpKind::Cast;
  op.to = to;
  return push(std::move(op), {a});
}

NodeId Graph::bitcast(NodeId a, DType to) {
  check_id("bitcast", a);
  if (dt_width(dtype(a)) != dt_width(to))
    throw Error(std::string("bitcast: width ") + dt_name(dtype(a)) + " != " + dt_name(to));
  Op op;
  op.kind = OpKind::Bitcast;
  op.to = to;
  return push(std::move(op), {a});
}

NodeId Graph::detach(NodeId a) {
  Op op;
  op.kind = OpKind::Detach;
  return push(std::move(op), {a});
}

// elementwise.rs:83-94: a 1-element const in `like`'s dtype, expanded to its shape.
NodeId Graph::scalar(NodeId like, float v) {
  check_id("scalar", like);
  DType dt = dtype(like);
  Shape ones(shape(like).size(), 1);
  std::vector<uint8_t> b(dt_width(dt));
  double x = static_cast<double>(v);
  switch (dt) {
    case DType::BOOL: b[0] = (x != 0.0); break;
    case DType::U8: { uint8_t t = sat_cast<uint8_t>(x); std::memcpy(b.data(), &t, 1); } break;
    case DType::U16: { uint16_t t = sat_cast<uint16_t>(x); std::memcpy(b.data(), &t, 2); } break;
    case DType::U32: { uint32_t t = sat_cast<uint32_t>(x); std::memcpy(b.data(), &t, 4); } break;
    case DType::U64: { uint64_t t = sat_cast<uint64_t>(x); std::memcpy(b.data(), &t, 8); } break;
    case DType::I8: { int8_t t = sat_cast<int8_t>(x); std::memcpy(b.data(), &t, 1); } break;
    case DType::I16: { int16_t t = sat_cast<int16_t>(x); std::memcpy(b.data(), &t, 2); } break;
    case DType::I32: { int32_t t = sat_cast<int32_t>(x); std::memcpy(b.data(), &t, 4); } break;
    case DType::I64: { int64_t t = sat_cast<int64_t>(x); std::memcpy(b.data(), &t, 8); } break;
    case DType::F8E4M3: b[0] = f32_to_f8e4m3(v); break;
    case DType::F8E5M2: b[0] = f32_to_f8e5m2(v); break;
    case DType::F16: { uint16_t t = f64_to_f16(x); std::memcpy(b.data(), &t, 2); } break;
    case DType::BF16: { uint16_t t = f64_to_bf16(x); std::memcpy(b.data(), &t, 2); } break;
    case DType::F32: std::memcpy(b.data(), &v, 4); break;
    case DType::F64: std::memcpy(b.data(), &x, 8); break;
    case DType::C64: { float c[2] = {v, 0.f}; std::memcpy(b.data(), c, 8); } break;
    case DType::C128: { double c[2] = {x, 0.0}; std::memcpy(b.data(), c, 16); } break;
  }
  NodeId c = constant_bytes(dt, b.data(), b.size(), ones);
  return expand(c, shape(like));
}

// ---------------- elementwise ----------------

NodeId Graph::add(NodeId a, NodeId b) {
  check_id("add", a); check_id("add", b);
  same_shape("add", a, b); same_dtype("add", a, b);
  require("add", a, dt_is_arith(dtype(a)), "numeric or complex");
  Op op; op.kind = OpKind::Add;
  return push(std::move(op), {a, b});
}
NodeId Graph::mul(NodeId a, NodeId b) {
  check_id("mul", a); check_id("mul", b);
  same_shape("mul", a, b); same_dtype("mul", a, b);
  require("mul", a, dt_is_arith(dtype(a)), "numeric or complex");
  Op op; op.kind = OpKind::Mul;
  return push(std::move(op), {a, b});
}
NodeId Graph::max(NodeId a, NodeId b) {
  check_id("max", a); check_id("max", b);
  same_shape("max", a, b); same_dtype("max", a, b);
  require("max", a, dt_is_numeric(dtype(a)), "numeric");
  Op op; op.kind = OpKind::Max;
  return push(std::move(op), {a, b});
}

static Op unary(OpKind k) { Op o; o.kind = k; return o; }

NodeId Graph::neg(NodeId a) {
  check_id("neg", a);
  require("neg", a, dt_is_signed(dtype(a)) || dt_is_complex(dtype(a)), "signed or complex");
  return push(unary(OpKind::Neg), {a});
}
NodeId Graph::recip(NodeId a) {
  check_id("recip", a);
  require("recip", a, dt_is_float(dtype(a)) || dt_is_complex(dtype(a)), "float or complex");
  return push(unary(OpKind::Recip), {a});
}
NodeId Graph::sqrt(NodeId a) {
  check_id("sqrt", a);
  require("sqrt", a, dt_is_float(dtype(a)) || dt_is_complex(dtype(a)), "float or complex");
  return push(unary(OpKind::Sqrt), {a});
}
NodeId Graph::exp2(NodeId a) {
  check_id("exp2", a);
  require("exp2", a, dt_is_float(dtype(a)) || dt_is_complex(dtype(a)), "float or complex");
  return push(unary(OpKind::Exp2), {a});
}
NodeId Graph::log2(NodeId a) {
  check_id("log2", a);
  require("log2", a, dt_is_float(dtype(a)) || dt_is_complex(dtype(a)), "float or complex");
  return push(unary(OpKind::Log2), {a});
}
NodeId Graph::sin(NodeId a) {
  check_id("sin", a);
  require("sin", a, dt_is_float(dtype(a)) || dt_is_complex(dtype(a)), "float or complex");
  return push(unary(OpKind::Sin), {a});
}
NodeId Graph::floor(NodeId a) {
  check_id("floor", a);
  require("floor", a, dt_is_float(dtype(a)), "float");
  return push(unary(OpKind::Floor), {a});
}

static bool is_bitwise(DType d) { return dt_is_int(d) || d == DType::BOOL; }

NodeId Graph::idiv(NodeId a, NodeId b) {
  check_id("idiv", a); check_id("idiv", b);
  same_shape("idiv", a, b); same_dtype("idiv", a, b);
  require("idiv", a, dt_is_int(dtype(a)), "integer");
  return push(unary(OpKind::IDiv), {a, b});
}
NodeId Graph::bit_and(NodeId a, NodeId b) {
  check_id("and", a); check_id("and", b);
  same_shape("and", a, b); same_dtype("and", a, b);
  require("and", a, is_bitwise(dtype(a)), "integer or bool");
  return push(unary(OpKind::And), {a, b});
}
NodeId Graph::bit_or(NodeId a, NodeId b) {
  check_id("or", a); check_id("or", b);
  same_shape("or", a, b); same_dtype("or", a, b);
  require("or", a, is_bitwise(dtype(a)), "integer or bool");
  return push(unary(OpKind::Or), {a, b});
}
NodeId Graph::bit_xor(NodeId a, NodeId b) {
  check_id("xor", a); check_id("xor", b);
  same_shape("xor", a, b); same_dtype("xor", a, b);
  require("xor", a, is_bitwise(dtype(a)), "integer or bool");
  return push(unary(OpKind::Xor), {a, b});
}
NodeId Graph::shl(NodeId a, NodeId b) {
  check_id("shl", a); check_id("shl", b);
  same_shape("shl", a, b); same_dtype("shl", a, b);
  require("shl", a, dt_is_int(dtype(a)), "integer");
  return push(unary(OpKind::Shl), {a, b});
}
NodeId Graph::shr(NodeId a, NodeId b) {
  check_id("shr", a); check_id("shr", b);
  same_shape("shr", a, b); same_dtype("shr", a, b);
  require("shr", a, dt_is_int(dtype(a)), "integer");
  return push(unary(OpKind::Shr), {a, b});
}
NodeId Graph::cmp_lt(NodeId a, NodeId b) {
  check_id("lt", a); check_id("lt", b);
  same_shape("lt", a, b); same_dtype("lt", a, b);
  require("lt", a, dt_is_numeric(dtype(a)), "numeric");
  return push(unary(OpKind::CmpLt), {a, b});
}
NodeId Graph::cmp_eq(NodeId a, NodeId b) {
  check_id("eq", a); check_id("eq", b);
  same_shape("eq", a, b); same_dtype("eq", a, b);
  return push(unary(OpKind::CmpEq), {a, b});
}
NodeId Graph::where(NodeId c, NodeId a, NodeId b) {
  check_id("where", c); check_id("where", a); check_id("where", b);
  if (dtype(c) != DType::BOOL) throw Error("where: condition must be BOOL");
  same_shape("where", c, a); same_shape("where", a, b); same_dtype("where", a, b);
  return push(unary(OpKind::Where), {c, a, b});
}

NodeId Graph::sub(NodeId a, NodeId b) { NodeId nb = neg(b); return add(a, nb); }
NodeId Graph::div(NodeId a, NodeId b) { NodeId rb = recip(b); return mul(a, rb); }
NodeId Graph::exp(NodeId a) {
  NodeId s = scalar(a, 1.44269504088896340736f);  // std::f32::consts::LOG2_E
  NodeId xs = mul(a, s);
  return exp2(xs);
}
NodeId Graph::ln(NodeId a) {
  NodeId l = log2(a);
  NodeId c = scalar(l, 0.693147180559945309417f);  // std::f32::consts::LN_2
  return mul(l, c);
}
NodeId Graph::relu(NodeId a) { NodeId z = scalar(a, 0.f); return max(a, z); }
// elementwise.rs:126-135: select(0 < x, 1, 0) + select(x < 0, -1, 0)
NodeId Graph::sign(NodeId a) {
  NodeId z = scalar(a, 0.f);
  NodeId pos = cmp_lt(z, a);
  NodeId ng = cmp_lt(a, z);
  NodeId one = scalar(a, 1.f);
  NodeId neg1 = scalar(a, -1.f);
  NodeId p = where(pos, one, z);
  NodeId n = where(ng, neg1, z);
  return add(p, n);
}
// elementwise.rs:164-168: ceil(x) = -floor(-x)
NodeId Graph::ceil(NodeId a) {
  NodeId nx = neg(a);
  NodeId f = floor(nx);
  return neg(f);
}
// elementwise.rs:171-175: round(x) = floor(x + 0.5)
NodeId Graph::round(NodeId a) {
  NodeId h = scalar(a, 0.5f);
  NodeId s = add(a, h);
  return floor(s);
}
NodeId Graph::square(NodeId a) { return mul(a, a); }
// trig.rs:16-20: cos(x) = sin(x + pi/2)
NodeId Graph::cos(NodeId a) {
  NodeId h = scalar(a, 1.57079632679489661923f);
  NodeId s = add(a, h);
  return sin(s);
}

NodeId Graph::tanh(NodeId a) {
  NodeId two = scalar(a, 2.0f);
  NodeId x2 = mul(a, two);
  NodeId s = sigmoid(x2);
  NodeId two2 = scalar(a, 2.0f);
  NodeId s2 = mul(s, two2);
  NodeId one = scalar(a, 1.0f);
  return sub(s2, one);
}
NodeId Graph::sigmoid(NodeId a) {
  NodeId na = neg(a);
  NodeId e = exp(na);
  NodeId one = scalar(a, 1.0f);
  NodeId d = add(one, e);
  return recip(d);
}
NodeId Graph::silu(NodeId a) {
  NodeId s = sigmoid(a);
  return mul(a, s);
}
NodeId Graph::gelu(NodeId a) {
  NodeId x2 = mul(a, a);
  NodeId x3 = mul(x2, a);
  NodeId c = scalar(a, 0.044715f);
  NodeId cx3 = mul(c, x3);
  NodeId inner = add(a, cx3);
  NodeId k = scalar(a, std::sqrt(2.0f / 3.14159265358979323846f));  // (2/pi).sqrt() in f32
  NodeId scaled = mul(k, inner);
  NodeId t = tanh(scaled);
  NodeId one = scalar(a, 1.0f);
  NodeId onep = add(one, t);
  NodeId half = scalar(a, 0.5f);
  NodeId hx = mul(half, a);
  return mul(hx, onep);
}

// attention.rs:9-36: x*cos + rotate_half(x)*sin over [.., S, D], angle[s,i] = s * 10000^(-2i/D),
// with cos = sin(angle + pi/2) and the tables built in f32 from two iotas.
NodeId Graph::rope(NodeId x) {
  check_id("rope", x);
  Shape xs = shape(x);
  size_t r = xs.size();
  if (r < 2) throw Error("rope: rank >= 2 required, got " + shape_str(xs));
  size_t s = xs[r - 2], d = xs[r - 1], half = d / 2;
  NodeId pos = iota({s, half}, 0, DType::F32);
  NodeId fi = iota({s, half}, 1, DType::F32);
  const float ln10000 = 9.21034049987792969f;  // 10000f32.ln(), the f32 nearest ln(10^4)
  NodeId c = scalar(fi, -2.0f * ln10000 / static_cast<float>(d));
  NodeId ic = mul(fi, c);
  NodeId theta = exp(ic);
  NodeId angle = mul(pos, theta);
  NodeId sin_h = sin(angle);
  NodeId hp = scalar(angle, 1.57079632679489661923f);  // FRAC_PI_2
  NodeId cos_arg = add(angle, hp);
  NodeId cos_h = sin(cos_arg);
  NodeId cos_full = concat_last(cos_h, cos_h, half);
  NodeId sin_full = concat_last(sin_h, sin_h, half);
  NodeId x1 = slice_last(x, 0, half);
  NodeId x2 = slice_last(x, half, d);
  NodeId nx2 = neg(x2);
  NodeId rot = concat_last(nx2, x1, half);
  NodeId cos_b = broadcast_2d_to(cos_full, xs);
  NodeId sin_b = broadcast_2d_to(sin_full, xs);
  NodeId a = mul(x, cos_b);
  NodeId b = mul(rot, sin_b);
  return add(a, b);
}

// attention.rs:39-50: [.., La] ++ [.., Lb] on the last axis as pad(a, right Lb) + pad(b, left La).
NodeId Graph::concat_last(NodeId a, NodeId b, size_t alen) {
  size_t r = shape(a).size();
  size_t blen = shape(b)[r - 1];
  std::vector<PadRange> pa(r, {0, 0}), pb(r, {0, 0});
  pa[r - 1] = {0, blen};
  pb[r - 1] = {alen, 0};
  NodeId ap = pad(a, pa);
  NodeId bp = pad(b, pb);
  return add(ap, bp);
}

// attention.rs:53-59
NodeId Graph::slice_last(NodeId a, size_t start, size_t end) {
  const Shape& sh = shape(a);
  std::vector<SliceRange> rg;
  for (size_t dim : sh) rg.push_back({0, dim, 1});
  rg.back() = {start, end, 1};
  return slice(a, rg);
}

// attention.rs:62-70: [A, B] -> [1, .., 1, A, B] -> target
NodeId Graph::broadcast_2d_to(NodeId t, const Shape& target) {
  const Shape& ts = shape(t);
  size_t r = target.size();
  Shape full(r, 1);
  full[r - 2] = ts[0];
  full[r - 1] = ts[1];
  NodeId tr = reshape(t, full);
  return expand(tr, target);
}

// random.rs:28-40 (Box-Muller over the `seed` and `seed ^ 0xD1B54A32D192ED03` streams)
NodeId Graph::randn(const Shape& shape, uint64_t seed) {
  NodeId u1 = rand_uniform(shape, seed);
  // clamp_min(u1, 1e-7) = max(u1, 1e-7)
  NodeId lo = scalar(u1, 1e-7f);
  u1 = max(u1, lo);
  NodeId u2 = rand_uniform(shape, seed ^ 0xD1B54A32D192ED03ull);
  NodeId lu = ln(u1);
  NodeId m2 = scalar(lu, -2.0f);
  NodeId r2 = mul(lu, m2);
  NodeId r = sqrt(r2);
  NodeId tau = scalar(u2, 6.28318530717958647692f);
  NodeId ang = mul(u2, tau);
  NodeId c = cos(ang);
  return mul(r, c);
}

NodeId Graph::rand_range(const Shape& shape, uint64_t seed, float lo, float hi) {
  NodeId u = rand_uniform(shape, seed);
  NodeId sc = scalar(u, hi - lo);
  NodeId su = mul(u, sc);
  NodeId off = scalar(su, lo);
  return add(su, off);
}

// ---------------- reductions ----------------

NodeId Graph::sum(NodeId a, size_t axis) {
  check_id("sum", a);
  reduce_axis_ok("sum", a, axis);
  require("sum", a, dt_is_arith(dtype(a)), "numeric or complex");
  Op op; op.kind = OpKind::Sum; op.axis = axis;
  return push(std::move(op), {a});
}
NodeId Graph::prod(NodeId a, size_t axis) {
  check_id("prod", a);
  reduce_axis_ok("prod", a, axis);
  require("prod", a, dt_is_arith(dtype(a)), "numeric or complex");
  Op op; op.kind = OpKind::Prod; op.axis = axis;
  return push(std::move(op), {a});
}
NodeId Graph::reduce_max(NodeId a, size_t axis) {
  check_id("reduce_max", a);
  reduce_axis_ok("reduce_max", a, axis);
  require("reduce_max", a, dt_is_numeric(dtype(a)), "numeric");
  Op op; op.kind = OpKind::ReduceMax; op.axis = axis;
  return push(std::move(op), {a});
}
NodeId Graph::argreduce(NodeId a, size_t axis, ArgKind k) {
  const char* nm = k == ArgKind::Max ? "argmax" : "argmin";
  check_id(nm, a);
  reduce_axis_ok(nm, a, axis);
  require(nm, a, dt_is_numeric(dtype(a)), "numeric");
  Op op; op.kind = OpKind::ArgReduce; op.axis = axis; op.arg = k;
  return push(std::move(op), {a});
}
// reduce.rs:38-43
NodeId Graph::broadcast_back(NodeId reduced, const Shape& full, size_t axis) {
  Shape keep = shape(reduced);
  keep.insert(keep.begin() + axis, 1);
  NodeId r = reshape(reduced, keep);
  return expand(r, full);
}
// reduce.rs:54-58: min over an axis is -reduce_max(-x)
NodeId Graph::reduce_min(NodeId a, size_t axis) {
  check_id("reduce_min", a);
  NodeId nx = neg(a);
  NodeId m = reduce_max(nx, axis);
  return neg(m);
}
// reduce.rs:115-124: m + ln(sum(exp(x - m))) with m = reduce_max(x)
NodeId Graph::logsumexp(NodeId a, size_t axis) {
  check_id("logsumexp", a);
  const Shape full = shape(a);
  NodeId m = reduce_max(a, axis);
  NodeId mb = broadcast_back(m, full, axis);
  NodeId sh = sub(a, mb);
  NodeId e = exp(sh);
  NodeId s = sum(e, axis);
  NodeId l = ln(s);
  return add(l, m);
}
// activation.rs:132-137: x - logsumexp(x) broadcast back
NodeId Graph::log_softmax(NodeId a, size_t axis) {
  check_id("log_softmax", a);
  const Shape full = shape(a);
  NodeId lse = logsumexp(a, axis);
  NodeId lb = broadcast_back(lse, full, axis);
  return sub(a, lb);
}
NodeId Graph::mean(NodeId a, size_t axis) {
  check_id("mean", a);
  reduce_axis_ok("mean", a, axis);
  float n = static_cast<float>(shape(a)[axis]);
  NodeId s = sum(a, axis);
  NodeId inv = scalar(s, 1.0f / n);
  return mul(s, inv);
}

// ---------------- nn ----------------

NodeId Graph::softmax(NodeId a, size_t axis) {
  check_id("softmax", a);
  if (axis >= shape(a).size())
    throw Error("softmax: axis " + std::to_string(axis) + " out of range for rank " + std::to_string(shape(a).size()));
  require("softmax", a, dt_is_float(dtype(a)), "float");
  Op op; op.kind = OpKind::Softmax; op.axis = axis;
  return push(std::move(op), {a});
}

NodeId Graph::rmsnorm(NodeId a, size_t axis, float eps) {
  check_id("rmsnorm", a);
  if (axis >= shape(a).size()) throw Error("rmsnorm: axis out of range");
  require("rmsnorm", a, dt_is_float(dtype(a)), "float");
  Op op; op.kind = OpKind::RmsNorm; op.axis = axis; op.eps = eps;
  return push(std::move(op), {a});
}

// attention.rs:83-90: fused Op::Sdpa only when the [..,S,S] f32 score buffer exceeds 1 GiB.
NodeId Graph::sdpa(NodeId q, NodeId k, NodeId v, bool causal) {
  check_id("sdpa", q); check_id("sdpa", k); check_id("sdpa", v);
  require("sdpa", q, dt_is_float(dtype(q)), "float");
  const Shape &qs = shape(q), &ks = shape(k), &vs = shape(v);
  if (qs.size() < 2) throw Error("sdpa: rank >= 2 required");
  size_t r = qs.size();
  size_t batch = 1;
  for (size_t i = 0; i + 2 < r; ++i) batch *= qs[i];
  size_t s = qs[r - 2];
  size_t score_bytes = batch * s * s * 4;
  if (qs == ks && qs == vs && score_bytes > (size_t(1) << 30)) return sdpa_fused(q, k, v, causal);
  return sdpa_decomposed(q, k, v, causal);
}

// attention.rs:97-113
NodeId Graph::sdpa_decomposed(NodeId q, NodeId k, NodeId v, bool causal) {
  check_id("sdpa_decomposed", q); check_id("sdpa_decomposed", k); check_id("sdpa_decomposed", v);
  Shape qs = shape(q);
  size_t r = qs.size();
  if (r < 2) throw Error("sdpa_decomposed: rank >= 2 required");
  size_t s = qs[r - 2], dh = qs[r - 1];
  std::vector<size_t> batch;
  for (size_t i = 0; i + 2 < r; ++i) batch.push_back(i);
  NodeId raw = dot_general(q, k, {r - 1}, {r - 1}, batch, batch);
  NodeId inv = scalar(raw, 1.0f / std::sqrt(static_cast<float>(dh)));
  NodeId scores = mul(raw, inv);
  if (causal) {
    DType dt = dtype(scores);
    NodeId bias = causal_bias(s, shape(scores));
    if (dt != DType::F32) bias = cast(bias, dt);
    scores = add(scores, bias);
  }
  NodeId attn = softmax(scores, r - 1);
  return dot_general(attn, v, {r - 1}, {r - 2}, batch, batch);
}

// attention.rs:120-133
NodeId Graph::sdpa_fused(NodeId q, NodeId k, NodeId v, bool causal) {
  check_id("sdpa_fused", q); check_id("sdpa_fused", k); check_id("sdpa_fused", v);
  const Shape &qs = shape(q), &ks = shape(k), &vs = shape(v);
  if (qs != ks || qs != vs)
    throw Error("sdpa_fused: q/k/v must share shape: " + shape_str(qs) + " " + shape_str(ks) + " " + shape_str(vs));
  size_t r = qs.size();
  if (r < 2 || qs[r - 1] == 0) throw Error("sdpa_fused: need rank>=2 with dh>0, got " + shape_str(qs));
  same_dtype("sdpa_fused", q, k);
  same_dtype("sdpa_fused", q, v);
  Op op; op.kind = OpKind::Sdpa; op.causal = causal;
  return push(std::move(op), {q, k, v});
}

// attention.rs:140-153: one f32 [S,S] const (0 on/below the diagonal, -inf above),
// reshaped to [1,..,1,S,S] and expanded to the score shape.
NodeId Graph::causal_bias(size_t s, const Shape& out_shape) {
  std::vector<float> data(s * s, 0.f);
  for (size_t i = 0; i < s; ++i)
    for (size_t j = i + 1; j < s; ++j) data[i * s + j] = -INFINITY;
  NodeId bias = constant_f32(data, {s, s});
  size_t rank = out_shape.size();
  Shape full(rank, 1);
  full[rank - 2] = s;
  full[rank - 1] = s;
  NodeId b = reshape(bias, full);
  return expand(b, out_shape);
}

// ---------------- movement ----------------

NodeId Graph::reshape(NodeId a, const Shape& s) {
  check_id("reshape", a);
  if (numel(shape(a)) != numel(s))
    throw Error("reshape: numel " + std::to_string(numel(shape(a))) + " -> " + std::to_string(numel(s)));
  Op op; op.kind = OpKind::Reshape; op.shape = s;
  return push(std::move(op), {a});
}
NodeId Graph::permute(NodeId a, const std::vector<size_t>& perm) {
  check_id("permute", a);
  std::vector<size_t> sorted = perm;
  std::sort(sorted.begin(), sorted.end());
  for (size_t i = 0; i < sorted.size(); ++i)
    if (sorted[i] != i || sorted.size() != shape(a).size())
      throw Error("permute: not a permutation of 0.." + std::to_string(shape(a).size()));
  if (sorted.size() != shape(a).size()) throw Error("permute: rank mismatch");
  Op op; op.kind = OpKind::Permute; op.perm = perm;
  return push(std::move(op), {a});
}
NodeId Graph::expand(NodeId a, const Shape& s) {
  check_id("expand", a);
  const Shape& from = shape(a);
  bool ok = from.size() == s.size();
  for (size_t i = 0; ok && i < s.size(); ++i) ok = (from[i] == s[i] || from[i] == 1);
  if (!ok) throw Error("expand: " + shape_str(from) + " -> " + shape_str(s));
  Op op; op.kind = OpKind::Expand; op.shape = s;
  return push(std::move(op), {a});
}
// view.rs:155-165 (NumPy rules: prepend ones, then expand)
NodeId Graph::broadcast_to(NodeId a, const Shape& s) {
  check_id("broadcast_to", a);
  Shape xs = shape(a);
  if (xs.size() > s.size()) throw Error("broadcast_to: rank " + shape_str(xs) + " -> " + shape_str(s));
  if (xs.size() < s.size()) {
    Shape p(s.size() - xs.size(), 1);
    p.insert(p.end(), xs.begin(), xs.end());
    a = reshape(a, p);
  }
  return expand(a, s);
}
NodeId Graph::transpose(NodeId a, size_t i, size_t j) {
  check_id("transpose", a);
  size_t r = shape(a).size();
  if (i >= r || j >= r) throw Error("transpose: axis out of range");
  std::vector<size_t> p(r);
  for (size_t t = 0; t < r; ++t) p[t] = t;
  std::swap(p[i], p[j]);
  return permute(a, p);
}
NodeId Graph::slice(NodeId a, const std::vector<SliceRange>& r) {
  check_id("slice", a);
  const Shape& s = shape(a);
  if (r.size() != s.size()) throw Error("slice: rank mismatch");
  for (size_t i = 0; i < r.size(); ++i)
    if (r[i].step == 0 || r[i].start > r[i].end || r[i].end > s[i]) throw Error("slice: bad range on axis " + std::to_string(i));
  Op op; op.kind = OpKind::Slice; op.ranges = r;
  return push(std::move(op), {a});
}
NodeId Graph::flip(NodeId a, const std::vector<size_t>& axes) {
  check_id("flip", a);
  for (size_t ax : axes)
    if (ax >= shape(a).size()) throw Error("flip: axis out of range");
  Op op; op.kind = OpKind::Flip; op.axes = axes;
  return push(std::move(op), {a});
}
NodeId Graph::pad(NodeId a, const std::vector<PadRange>& p) {
  check_id("pad", a);
  if (p.size() != shape(a).size()) throw Error("pad: rank mismatch");
  Op op; op.kind = OpKind::Pad; op.pads = p;
  return push(std::move(op), {a});
}

// ---------------- contraction ----------------

static void check_axes(const std::vector<size_t>& axes, size_t rank) {
  for (size_t k = 0; k < axes.size(); ++k) {
    if (axes[k] >= rank)
      throw Error("dot_general: axis " + std::to_string(axes[k]) + " out of range for rank " + std::to_string(rank));
    for (size_t j = 0; j < k; ++j)
      if (axes[j] == axes[k]) throw Error("dot_general: axis " + std::to_string(axes[k]) + " used twice");
  }
}

NodeId Graph::dot_general(NodeId a, NodeId b, const std::vector<size_t>& lc, const std::vector<size_t>& rc,
                          const std::vector<size_t>& lb, const std::vector<size_t>& rb) {
  check_id("dot_general", a); check_id("dot_general", b);
  const Shape sa = shape(a), sb = shape(b);
  same_dtype("dot_general", a, b);
  require("dot_general", a, dt_is_arith(dtype(a)), "numeric or complex");
  if (lc.size() != rc.size()) throw Error("dot_general: contract count mismatch");
  if (lb.size() != rb.size()) throw Error("dot_general: batch count mismatch");
  std::vector<size_t> aa(lb), ba(rb);
  aa.insert(aa.end(), lc.begin(), lc.end());
  ba.insert(ba.end(), rc.begin(), rc.end());
  check_axes(aa, sa.size());
  check_axes(ba, sb.size());
  for (size_t i = 0; i < lb.size(); ++i)
    if (sa[lb[i]] != sb[rb[i]])
      throw Error("dot_general: batch dim " + std::to_string(sa[lb[i]]) + " vs " + std::to_string(sb[rb[i]]));
  for (size_t i = 0; i < lc.size(); ++i)
    if (sa[lc[i]] != sb[rc[i]])
      throw Error("dot_general: contract dim " + std::to_string(sa[lc[i]]) + " vs " + std::to_string(sb[rc[i]]));
  Op op; op.kind = OpKind::DotGeneral; op.lc = lc; op.rc = rc; op.lb = lb; op.rb = rb;
  return push(std::move(op), {a, b});
}

// graph/ops/core/contract.rs:49-115: the reference's record-time checks, in its order.
NodeId Graph::quant_matmul(NodeId act, NodeId qw, NodeId scales, NodeId mins, int bits, size_t group_size) {
  const char* nm = "quant_matmul";
  check_id(nm, act); check_id(nm, qw); check_id(nm, scales);
  if (mins != kNoNode) check_id(nm, mins);
  const Shape &sa = shape(act), &sq = shape(qw);
  if (sa.size() != 2 || sq.size() != 2)
    throw Error(std::string(nm) + ": act rank " + std::to_string(sa.size()) + ", qweight rank " +
                std::to_string(sq.size()) + ": both must be rank-2");
  if (dtype(qw) != DType::U8) throw Error(std::string(nm) + ": qweight must be U8, got " + dt_name(dtype(qw)));
  if (dtype(scales) != DType::F16) throw Error(std::string(nm) + ": scales must be F16, got " + dt_name(dtype(scales)));
  if (mins != kNoNode && dtype(mins) != DType::F16)
    throw Error(std::string(nm) + ": mins must be F16, got " + dt_name(dtype(mins)));
  if (!dt_is_float(dtype(act))) throw Error(std::string(nm) + ": act must be float, got " + dt_name(dtype(act)));
  const size_t k = sa[1], n = sq[0];
  if (!(bits == 2 || bits == 4 || bits == 8))
    throw Error(std::string(nm) + ": bits " + std::to_string(bits) + " must be 2, 4, or 8");
  if (group_size == 0 || k % group_size != 0)
    throw Error(std::string(nm) + ": K " + std::to_string(k) + " must be a nonzero multiple of group_size " +
                std::to_string(group_size));
  if (sq[1] * 8 != k * (size_t)bits)
    throw Error(std::string(nm) + ": qweight cols " + std::to_string(sq[1]) + " must equal K*bits/8 = " +
                std::to_string(k) + "*" + std::to_string(bits) + "/8");
  const size_t want = n * (k / group_size);
  if (numel(shape(scales)) != want)
    throw Error(std::string(nm) + ": scales must have N*K/group_size = " + std::to_string(want) + " entries");
  if (mins != kNoNode && numel(shape(mins)) != want)
    throw Error(std::string(nm) + ": mins must have N*K/group_size = " + std::to_string(want) + " entries");
  Op op;
  op.kind = OpKind::QuantMatmul;
  op.qbits = bits;
  op.qgroup = group_size;
  op.qsym = mins == kNoNode;
  std::vector<NodeId> src = {act, qw, scales};
  if (mins != kNoNode) src.push_back(mins);
  return push(std::move(op), std::move(src));
}

// capi/ops/contract.rs:11-13: ku_matmul = 2D dot_general contracting a's axis 1 with b's axis 0.
NodeId Graph::matmul(NodeId a, NodeId b) {
  check_id("matmul", a); check_id("matmul", b);
  if (shape(a).size() != 2 || shape(b).size() != 2) throw Error("matmul: 2D operands required");
  return dot_general(a, b, {1}, {0}, {}, {});
}

// ---------------- inspection ----------------

std::vector<NodeId> reachable_multi(const Graph& g, const std::vector<NodeId>& roots) {
  std::vector<NodeId> order;
  std::unordered_set<NodeId> seen;
  std::vector<std::pair<NodeId, bool>> stack;
  for (size_t i = roots.size(); i-- > 0;) stack.push_back({roots[i], false});
  while (!stack.empty()) {
    auto [id, expanded] = stack.back();
    stack.pop_back();
    if (expanded) { order.push_back(id); continue; }
    if (!seen.insert(id).second) continue;
    stack.push_back({id, true});
    for (NodeId s : g.node(id).src)
      if (!seen.count(s)) stack.push_back({s, false});
  }
  return order;
}

static std::string label(const Node& n) {
  std::ostringstream o;
  const Op& op = n.op;
  switch (op.kind) {
    case OpKind::Const: o << "Const" << shape_str(op.shape); break;
    case OpKind::Input: o << "Input" << shape_str(op.shape); break;
    case OpKind::Cast: o << "Cast { to: " << dt_name(op.to) << " }"; break;
    case OpKind::Bitcast: o << "Bitcast { to: " << dt_name(op.to) << " }"; break;
    case OpKind::Sum: case OpKind::Prod: case OpKind::ReduceMax: case OpKind::Softmax:
      o << op_name(op.kind) << " { axis: " << op.axis << " }"; break;
    case OpKind::ArgReduce:
      o << "ArgReduce { axis: " << op.axis << ", kind: " << (op.arg == ArgKind::Max ? "Max" : "Min") << " }"; break;
    case OpKind::Reshape: o << "Reshape { shape: " << shape_str(op.shape) << " }"; break;
    case OpKind::Expand: o << "Expand { shape: " << shape_str(op.shape) << " }"; break;
    case OpKind::Permute: o << "Permute { perm: " << shape_str(op.perm) << " }"; break;
    case OpKind::Sdpa: o << "Sdpa { causal: " << (op.causal ? "true" : "false") << " }"; break;
    case OpKind::QuantMatmul:
      o << "QuantMatmul { bits: " << op.qbits << ", group_size: " << op.qgroup << ", symmetric: "
        << (op.qsym ? "true" : "false") << " }";
      break;
    case OpKind::DotGeneral:
      o << "DotGeneral { lhs_contract: " << shape_str(op.lc) << ", rhs_contract: " << shape_str(op.rc)
        << ", lhs_batch: " << shape_str(op.lb) << ", rhs_batch: " << shape_str(op.rb) << " }";
      break;
    default: o << op_name(op.kind);
  }
  return o.str();
}

std::string dump(const Graph& g, NodeId root) {
  std::ostringstream o;
  for (NodeId id : reachable_multi(g, {root})) {
    const Node& n = g.node(id);
    o << "%" << id << " = " << label(n) << "(";
    for (size_t i = 0; i < n.src.size(); ++i) o << (i ? ", " : "") << "%" << n.src[i];
    o << ") : " << shape_str(n.shape) << "\n";
  }
  return o.str();
}

}  // namespace ku
