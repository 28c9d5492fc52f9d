// HIP source generation for line regions (kernel family 1: fused pointwise/reduce, and
// family 3: the one-pass softmax with its argmax epilogue).
//
// A region iterates a shape S. Without a reduction axis it is a flat elementwise kernel
// (each thread owns V consecutive elements, 128-bit loads/stores where the layout allows).
// With an axis it is a line kernel: TPL threads own one line of S along the axis, hold
// the line's loaded values in registers across phases, fold each reduction level with a
// wave64 butterfly (+ an LDS combine across waves) and store every output in the same
// pass. Per-primitive rounding of f16/bf16/fp8 values matches the oracle
// (kurumi_core/src/dtype/traits/float.rs:8-72,132-161): each op computes in f32 and rounds.
// Reductions of low-precision floats accumulate in f32 and round once
// (interp/reduce.rs:89-106). ArgReduce keeps the oracle's first-index tie rule and its NaN
// behaviour (interp/reduce.rs:18-65). The reference's Metal emitters this replaces are
// kurumi_metal/src/backend/fuse/emit.rs:80-142.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstdio>
#include <functional>
#include <map>
#include <set>
#include <sstream>

#include "device_prelude.h"
#include "plan.h"

namespace ku::hipbk {

namespace {

const char* stype(DType d) {  // storage type
  switch (d) {
    case DType::BOOL: case DType::U8: case DType::F8E4M3: case DType::F8E5M2: return "u8";
    case DType::U16: case DType::F16: case DType::BF16: return "u16";
    case DType::U32: return "u32";
    case DType::U64: return "u64";
    case DType::I8: return "i8";
    case DType::I16: return "i16";
    case DType::I32: return "i32";
    case DType::I64: return "i64";
    case DType::F32: return "float";
    case DType::F64: return "double";
    default: throw Error(std::string("kurumi_hip: dtype ") + dt_name(d) + " is not supported on device");
  }
}
const char* ctype(DType d) {  // compute type
  switch (d) {
    case DType::BOOL: return "bool";
    case DType::F8E4M3: case DType::F8E5M2: case DType::F16: case DType::BF16: case DType::F32: return "float";
    case DType::F64: return "double";
    default: return stype(d);
  }
}
const char* utype(DType d) {  // unsigned twin for wrapping arithmetic
  switch (d) {
    case DType::U8: case DType::I8: return "u8";
    case DType::U16: case DType::I16: return "u16";
    case DType::U32: case DType::I32: return "u32";
    case DType::U64: case DType::I64: return "u64";
    default: return "u32";
  }
}
int bits(DType d) { return (int)dt_width(d) * 8; }
bool fvalued(DType d) { return d == DType::F32 || dt_is_lowp(d); }

std::string ld(DType d, const std::string& raw) {
  switch (d) {
    case DType::BOOL: return "(" + raw + " != 0)";
    case DType::F16: return "f16_ld(" + raw + ")";
    case DType::BF16: return "bf16_ld(" + raw + ")";
    case DType::F8E4M3: return "f8e4m3_ld(" + raw + ")";
    case DType::F8E5M2: return "f8e5m2_ld(" + raw + ")";
    default: return raw;
  }
}
std::string st(DType d, const std::string& v) {
  switch (d) {
    case DType::BOOL: return "(u8)(" + v + ")";
    case DType::F16: return "f16_st(" + v + ")";
    case DType::BF16: return "bf16_st(" + v + ")";
    case DType::F8E4M3: return "f8e4m3_st(" + v + ")";
    case DType::F8E5M2: return "f8e5m2_st(" + v + ")";
    default: return v;
  }
}
std::string rnd(DType d, const std::string& v) {
  switch (d) {
    case DType::F16: return "rf16(" + v + ")";
    case DType::BF16: return "rbf16(" + v + ")";
    case DType::F8E4M3: return "rf8e4m3(" + v + ")";
    case DType::F8E5M2: return "rf8e5m2(" + v + ")";
    default: return v;
  }
}

// cast with the reference's through-f64 semantics
std::string cast_expr(DType from, DType to, const std::string& x) {
  if (from == to) return x;
  bool ffrom = fvalued(from);
  std::string dx = "((double)(" + x + "))";
  switch (to) {
    case DType::F32:
      // the reference widens through f64, which quiets a signalling NaN
      if (ffrom) return "quiet_nan(" + x + ")";
      return "((float)" + dx + ")";
    case DType::F64: return dx;
    case DType::BF16: return ffrom ? "rbf16(" + x + ")" : "rbf16_d(" + dx + ")";
    case DType::F16: return ffrom ? "rf16(" + x + ")" : "rf16_d(" + dx + ")";
    case DType::F8E4M3: return ffrom ? "rf8e4m3(" + x + ")" : "rf8e4m3((float)" + dx + ")";
    case DType::F8E5M2: return ffrom ? "rf8e5m2(" + x + ")" : "rf8e5m2((float)" + dx + ")";
    case DType::BOOL: return "(" + dx + " != 0.0)";
    default: return std::string("sat_int<") + stype(to) + ">(" + dx + ")";
  }
}

std::string flt_lit(DType acc, double v) {
  std::ostringstream o;
  o.precision(17);
  if (std::isinf(v)) return acc == DType::F64 ? (v > 0 ? "(double)INFINITY" : "(-(double)INFINITY)") : (v > 0 ? "INFINITY" : "(-INFINITY)");
  o << v;
  std::string s = o.str();
  if (s.find_first_of(".e") == std::string::npos) s += ".0";
  return acc == DType::F64 ? s : s + "f";
}

std::string int_min(DType d) {
  switch (d) {
    case DType::I8: return "(i8)-128";
    case DType::I16: return "(i16)-32768";
    case DType::I32: return "(i32)(-2147483647 - 1)";
    case DType::I64: return "(i64)(-9223372036854775807ll - 1)";
    default: return std::string("(") + stype(d) + ")0";
  }
}
std::string int_max(DType d) {
  switch (d) {
    case DType::I8: return "(i8)127";
    case DType::I16: return "(i16)32767";
    case DType::I32: return "(i32)2147483647";
    case DType::I64: return "(i64)9223372036854775807ll";
    case DType::U8: return "(u8)255";
    case DType::U16: return "(u16)65535";
    case DType::U32: return "(u32)4294967295u";
    case DType::U64: return "(u64)18446744073709551615ull";
    default: return "0";
  }
}

bool is_red(int k) {
  return k == (int)OpKind::Sum || k == (int)OpKind::Prod || k == (int)OpKind::ReduceMax || k == (int)OpKind::ArgReduce;
}

struct Gen {
  const Region& R;
  const std::vector<Slot>& slots;
  int index;
  std::ostringstream o;
  int rank = 0, a = -1;
  bool flat = true;
  int V = 1, TPL = 1, NC = 1, WG = 256, GPW = 1, FK = 1;
  uint64_t lines = 1, L = 1, N = 1;
  bool idx64 = false;
  std::vector<int> param_slots;
  std::map<int, int> slot_param;
  std::vector<bool> leaf_vec;
  int P = 0;  // reduction levels
  std::vector<int> store_phase;    // per node: phase in which a FULL output is stored (0 none)
  std::map<int, int> out_slot;     // rnode -> slot
  std::vector<std::set<int>> need; // per phase (1..P+1): FULL nodes computed in that phase
  std::set<int> cached;
  std::vector<int> first_phase;    // per node: first phase computing it
  bool has_final = false;
  bool unroll = false;
  int min_waves = 1;  // amdgpu_waves_per_eu lower bound of a line kernel

  Gen(const Region& r, const std::vector<Slot>& s, int i) : R(r), slots(s), index(i) {}

  int param(int slot) {
    auto it = slot_param.find(slot);
    if (it != slot_param.end()) return it->second;
    param_slots.push_back(slot);
    slot_param[slot] = (int)param_slots.size() - 1;
    return (int)param_slots.size() - 1;
  }
  const RNode& node(int i) const { return R.nodes[i]; }
  bool full(int i) const { return R.nodes[i].space == Space::Full; }
  // An f32 division by a line value whose every consumer rounds to a 16- or 8-bit float:
  // computed as x * (1 / d) with the reciprocal taken once per line. The product differs from
  // the quotient by at most one f32 ulp, which moves the narrow result only when it lies
  // within 2^-24 of a rounding boundary (1 narrow ulp then).
  bool div_by_line_recip(int ni) const {
    const RNode& n = R.nodes[ni];
    if (n.kind != RK_DIV || n.dtype != DType::F32 || flat || full(n.in[1])) return false;
    bool any = false;
    for (size_t i = 0; i < R.nodes.size(); ++i)
      for (int j : R.nodes[i].in)
        if (j == ni) {
          const RNode& c = R.nodes[i];
          if (c.kind != (int)OpKind::Cast || !dt_is_lowp(c.to)) return false;
          any = true;
        }
    for (auto& op : R.outputs)
      if (op.first == ni) return false;
    return any;
  }
  // Every consumer of node ni is IEEE arithmetic that turns a signalling NaN operand into the
  // same quiet NaN by itself (and ni is not stored), so a widening cast need not quiet first.
  bool consumers_quiet(int ni) const {
    for (auto& op : R.outputs)
      if (op.first == ni) return false;
    for (size_t i = 0; i < R.nodes.size(); ++i)
      for (int j : R.nodes[i].in)
        if (j == ni) {
          int k = R.nodes[i].kind;
          bool q = k == (int)OpKind::Add || k == (int)OpKind::Mul || k == (int)OpKind::Recip ||
                   k == (int)OpKind::Sqrt || k == (int)OpKind::Exp2 || k == (int)OpKind::Log2 ||
                   k == (int)OpKind::Sin || k == (int)OpKind::Floor || k == (int)OpKind::Sum ||
                   k == (int)OpKind::Prod || k == RK_DIV || k == RK_EXP || k == RK_SQRT_ADD_EPS ||
                   (k == (int)OpKind::Cast && (R.nodes[i].to == DType::BF16 || R.nodes[i].to == DType::F16));
          if (!q) return false;
        }
    return true;
  }
  bool needs_line_recip(int li) const {
    for (size_t i = 0; i < R.nodes.size(); ++i)
      if (R.nodes[i].kind == RK_DIV && R.nodes[i].in[1] == li && div_by_line_recip((int)i)) return true;
    return false;
  }
  std::string ix() const { return idx64 ? "u64" : "u32"; }

  // value of node i at element j (FULL) or as a line scalar (LINE)
  std::string val(int i, const std::string& j) const {
    if (full(i)) return "f" + std::to_string(i) + "[" + j + "]";
    return "s" + std::to_string(i);
  }

  std::string op_expr(int ni, const std::string& j) const;
  void plan_layout();
  void schedule();
  void emit_leaf_load(int ni, const std::string& c_expr);
  void emit_leaf_convert(int ni);
  // argmax/argmin index type along the line (32-bit unless the line is that long)
  // Non-temporal line-kernel accesses (bit 0 stores, bit 1 loads): a line is read once and its
  // outputs written once, so neither should displace reused data in L2 / MALL. Stores always;
  // loads only in regions that also stream a full-size output (a reduce-only region, which
  // reads far more than it writes, measured slower with non-temporal loads).
  // KURUMI_HIP_NT overrides.
  // Non-temporal accesses of flat (elementwise) kernels, bit 1 = stores, bit 2 = loads.
  // Streaming stores are non-temporal by default (measured: copy 6.21 -> 6.35 TB/s, rope 67 ->
  // 82 % of peak, SwiGLU gate 67 -> 80 %); non-temporal loads help a pure copy but slow the
  // kernels that re-read an input through the cache (rope's halves). KURUMI_HIP_FLAT_NT overrides.
  int flat_nt() const {
    static const int v = [] {
      const char* e = std::getenv("KURUMI_HIP_FLAT_NT");
      return e ? std::atoi(e) : 1;
    }();
    return v;
  }
  int nt_mode() const {
    static const int forced = [] {
      const char* e = std::getenv("KURUMI_HIP_NT");
      return e ? std::atoi(e) : -1;
    }();
    if (forced >= 0) return forced;
    // non-temporal stores always; non-temporal loads too when a full-size output is written and
    // lines are long (measured: the 128 KB rows of the f32 softmax gain ~2 %, the 8 KB rows of a
    // bf16 rmsnorm lose ~5 % with them)
    bool full_out = false;
    for (auto& op : R.outputs)
      if (full(op.first)) full_out = true;
    size_t wmax = 1;
    for (auto& l : R.leaves) wmax = std::max(wmax, dt_width(l.dtype));
    bool long_lines = a >= 0 && (uint64_t)L * wmax >= 32768;
    return full_out && long_lines ? 3 : 1;
  }
  // a vectorised bf16 leaf is loaded and kept as packed 32-bit words
  bool bf16_words(int c) const {
    const RNode& cn = node(c);
    return cn.kind == RK_LEAF && R.leaves[cn.leaf].dtype == DType::BF16 && V % 2 == 0 && leaf_vec[cn.leaf] &&
           !R.leaves[cn.leaf].view.padded() && !R.leaves[cn.leaf].imm;
  }
  // 16-bit leaves are cached two to a 32-bit register. (bf16 intermediates could be too -- every
  // bf16 value is carried bf16-exact -- but the pack/unpack VALU cost more than the registers
  // saved in the bf16 softmax, which is VALU-bound; they are cached as f32.)
  bool packed_cache(int c) const {
    const RNode& cn = node(c);
    if (V % 2 != 0) return false;
    return cn.kind == RK_LEAF && dt_width(R.leaves[cn.leaf].dtype) == 2;
  }
  bool bf16_packed(int c) const {
    const RNode& cn = node(c);
    return packed_cache(c) && (cn.kind == RK_LEAF ? R.leaves[cn.leaf].dtype : cn.dtype) == DType::BF16;
  }
  std::string aix() const { return L >= ((uint64_t)1 << 31) ? "i64" : "i32"; }
  std::string aix_none() const { return L >= ((uint64_t)1 << 31) ? "(i64)9223372036854775807ll" : "(i32)2147483647"; }
  void emit_full_node(int ni, int phase, const std::string& c_expr);
  void emit_line_node(int ni);
  void emit_red_init(int ni);
  void emit_red_update(int ni, const std::string& k_expr, const std::string& j);
  void emit_red_chunk_arg(int ni);
  void emit_red_finish(int ni, int phase);
  // A float ArgReduce over vector chunks folds per chunk: the chunk's extreme (one maxNum/minNum
  // tree), one strict comparison with the running best, and a conditional copy of the chunk's
  // values; the index inside the winning chunk is found once per thread at the end. Per element
  // that is about a third of the compare-and-select-index work of a per-element fold.
  bool chunk_arg(int ni) const {
    const RNode& n = node(ni);
    return n.kind == (int)OpKind::ArgReduce && V >= 2 && fvalued(node(n.in[0]).dtype) && !flat;
  }
  bool chunk_arg_packed(int ni) const { return chunk_arg(ni) && node(node(ni).in[0]).dtype == DType::BF16 && V % 2 == 0; }
  std::string leaf_base(int leaf) const;
  std::string generate(RegionCode* rc);
  std::string finish(const std::string& prefix, RegionCode* rc) {
    std::string src = o.str();
    uint64_t h = 1469598103934665603ull;
    for (unsigned char ch : src) h = (h ^ ch) * 1099511628211ull;
    char hex[16];
    std::snprintf(hex, sizeof hex, "%06llx", (unsigned long long)(h & 0xffffff));
    rc->entry = prefix + "_" + hex;
    size_t at = src.find("KU_ENTRY_PLACEHOLDER");
    src.replace(at, std::string("KU_ENTRY_PLACEHOLDER").size(), rc->entry);
    return src;
  }
};

std::string Gen::op_expr(int ni, const std::string& j) const {
  const RNode& n = node(ni);
  DType d = n.dtype;
  auto in = [&](int t) { return val(n.in[t], j); };
  auto indt = [&](int t) { return node(n.in[t]).dtype; };
  bool fl = fvalued(d), f64 = d == DType::F64;
  std::string U = utype(d), T = stype(d);
  switch (n.kind) {
    case (int)OpKind::Add:
      if (fl || f64) return rnd(d, "(" + in(0) + " + " + in(1) + ")");
      return "(" + T + ")((" + U + ")" + in(0) + " + (" + U + ")" + in(1) + ")";
    case (int)OpKind::Mul:
      if (fl || f64) return rnd(d, "(" + in(0) + " * " + in(1) + ")");
      return "(" + T + ")((" + U + ")" + in(0) + " * (" + U + ")" + in(1) + ")";
    case (int)OpKind::Max:
      if (fl) return "fmaxf(" + in(0) + ", " + in(1) + ")";
      if (f64) return "fmax(" + in(0) + ", " + in(1) + ")";
      return "(" + in(0) + " > " + in(1) + " ? " + in(0) + " : " + in(1) + ")";
    case (int)OpKind::Neg:
      if (fl || f64) return "(-" + in(0) + ")";
      return "(" + T + ")(0 - (" + U + ")" + in(0) + ")";
    case (int)OpKind::Recip:
      if (f64) return "(1.0 / " + in(0) + ")";
      // per-element results rounded to 16 or 8 bits right away: v_rcp_f32 (1 ulp) instead of the
      // correctly rounded f32 division, as for exp2 below (a once-per-line value keeps the division)
      if (n.space == Space::Full && (d == DType::BF16 || d == DType::F16 || d == DType::F8E4M3 || d == DType::F8E5M2))
        return rnd(d, "__builtin_amdgcn_rcpf(" + in(0) + ")");
      return rnd(d, "(1.0f / " + in(0) + ")");
    case (int)OpKind::Sqrt: return f64 ? "sqrt(" + in(0) + ")" : rnd(d, "sqrtf(" + in(0) + ")");
    case (int)OpKind::Exp2:
      if (f64) return "exp2(" + in(0) + ")";
      // rounded to 16 or 8 bits right away: the bare v_exp_f32 (1 ulp; results below 2^-126,
      // which would be bf16 denormals, come out as zero) instead of the denormal-safe exp2f
      if (d == DType::BF16 || d == DType::F16 || d == DType::F8E4M3 || d == DType::F8E5M2)
        return rnd(d, "__builtin_amdgcn_exp2f(" + in(0) + ")");
      return rnd(d, "exp2f(" + in(0) + ")");
    case (int)OpKind::Log2: return f64 ? "log2(" + in(0) + ")" : rnd(d, "log2f(" + in(0) + ")");
    case (int)OpKind::Sin: return f64 ? "sin(" + in(0) + ")" : rnd(d, "sinf(" + in(0) + ")");
    case (int)OpKind::Floor: return f64 ? "floor(" + in(0) + ")" : rnd(d, "floorf(" + in(0) + ")");
    case (int)OpKind::IDiv:
      if (dt_is_unsigned(d)) return "(" + in(1) + " == 0 ? (" + T + ")0 : (" + T + ")(" + in(0) + " / " + in(1) + "))";
      return "(" + in(1) + " == 0 ? (" + T + ")0 : (" + in(1) + " == -1 ? (" + T + ")(0 - (" + U + ")" + in(0) +
             ") : (" + T + ")(" + in(0) + " / " + in(1) + ")))";
    case (int)OpKind::And: return d == DType::BOOL ? "(" + in(0) + " && " + in(1) + ")" : "(" + T + ")(" + in(0) + " & " + in(1) + ")";
    case (int)OpKind::Or: return d == DType::BOOL ? "(" + in(0) + " || " + in(1) + ")" : "(" + T + ")(" + in(0) + " | " + in(1) + ")";
    case (int)OpKind::Xor: return d == DType::BOOL ? "(" + in(0) + " != " + in(1) + ")" : "(" + T + ")(" + in(0) + " ^ " + in(1) + ")";
    case (int)OpKind::Shl:
      return "(" + T + ")((" + U + ")" + in(0) + " << ((" + U + ")" + in(1) + " & " + std::to_string(bits(d) - 1) + "))";
    case (int)OpKind::Shr:
      return "(" + T + ")(" + in(0) + " >> ((" + U + ")" + in(1) + " & " + std::to_string(bits(d) - 1) + "))";
    case (int)OpKind::CmpLt: return "(" + in(0) + " < " + in(1) + ")";
    case (int)OpKind::CmpEq: return "(" + in(0) + " == " + in(1) + ")";
    case (int)OpKind::Where: return "(" + in(0) + " ? " + in(1) + " : " + in(2) + ")";
    case (int)OpKind::Cast:
      if (n.to == DType::F32 && dt_is_lowp(indt(0)) && consumers_quiet(ni)) return in(0);
      return cast_expr(indt(0), n.to, in(0));
    case (int)OpKind::Bitcast: {
      DType s = indt(0);
      std::string raw = std::string("__builtin_bit_cast(") + stype(n.to) + ", (" + stype(s) + ")" + st(s, in(0)) + ")";
      if (s == DType::BOOL || n.to == DType::BOOL) raw = std::string("(") + stype(n.to) + ")" + st(s, in(0));
      return ld(n.to, raw);
    }
    case RK_DIV:
      if (div_by_line_recip(ni)) return "(" + in(0) + " * s" + std::to_string(n.in[1]) + "_inv)";
      return "(" + in(0) + " / " + in(1) + ")";
    case RK_EXP: return f64 ? "exp(" + in(0) + ")" : "expf(" + in(0) + ")";
    case RK_SQRT_ADD_EPS: {
      std::string len = flt_lit(d, (double)n.axis), eps = flt_lit(d, (double)n.eps);
      return f64 ? "sqrt(" + in(0) + " / " + len + " + " + eps + ")" : "sqrtf(" + in(0) + " / " + len + " + " + eps + ")";
    }
    default:
      throw Error(std::string("kurumi_hip codegen: unsupported region op ") + op_name((OpKind)n.kind));
  }
}

// Decide flat vs line layout, vector width, threads per line, chunks per thread.
void Gen::plan_layout() {
  rank = (int)R.S.size();
  a = R.axis;
  N = numel(R.S);
  flat = a < 0;
  size_t maxoff = N;
  for (auto& l : R.leaves) {
    int64_t hi = l.view.offset, lo = l.view.offset;
    bool empty = false;
    for (size_t d = 0; d < l.view.shape.size(); ++d) {
      // addressed coordinates: the pad window of a padded view, else the whole axis
      int64_t c0 = l.view.padded() ? l.view.wlo[d] : 0;
      int64_t c1 = l.view.padded() ? l.view.whi[d] - 1 : (int64_t)l.view.shape[d] - 1;
      if (c1 < c0) { empty = true; break; }
      int64_t a0 = c0 * l.view.strides[d], a1 = c1 * l.view.strides[d];
      hi += std::max(a0, a1);
      lo += std::min(a0, a1);
    }
    if (empty) continue;
    maxoff = std::max<size_t>(maxoff, (size_t)std::max<int64_t>(hi, 0) + 1);
    if (lo < 0) maxoff = std::max<size_t>(maxoff, (size_t)1 << 40);
  }
  idx64 = maxoff >= ((size_t)1 << 31);
  int vecaxis = flat ? rank - 1 : a;
  uint64_t inner = 1;
  if (!flat)
    for (int d = a + 1; d < rank; ++d) inner *= R.S[d];
  L = flat ? R.S[rank - 1] : R.S[a];
  // lines: the iteration shape without its line axis (still counted when that axis is empty: a
  // reduction over a zero-length axis writes its identity to every line)
  lines = 1;
  for (int d = 0; d < rank; ++d)
    if (d != (flat ? rank - 1 : a)) lines *= R.S[d];
  // vector width: 16 bytes of the narrowest streamed type, only along a contiguous last axis
  int minw = 8;
  bool contiguous_axis = flat || inner == 1;
  for (auto& l : R.leaves)
    if (l.view.strides[vecaxis] != 0) minw = std::min<int>(minw, (int)dt_width(l.dtype));
  // A line region's V and TPL fix the order its reductions add in, so they depend only on what
  // the reduced values are computed from (leaves, line length, the region's structure), never
  // on which values are stored: a node evaluated alone and within eval_many over several roots
  // then gets the same bits (kurumi_core/tests/engine.rs:224-243). Flat regions (no reductions)
  // size their vectors by their outputs too.
  if (flat)
    for (auto& op : R.outputs) minw = std::min<int>(minw, (int)dt_width(node(op.first).dtype));
  V = contiguous_axis ? std::min(8, 16 / std::max(minw, 1)) : 1;
  while (V > 1 && (L % (uint64_t)V) != 0) V /= 2;
  leaf_vec.assign(R.leaves.size(), false);
  for (size_t i = 0; i < R.leaves.size(); ++i) {
    const View& v = R.leaves[i].view;
    // a padded view vectorises when its window on the vector axis is whole vectors (each
    // vector then lies entirely inside or entirely outside)
    bool win_ok = !v.padded() || (v.wlo[vecaxis] % V == 0 && v.whi[vecaxis] % V == 0);
    bool ok = V > 1 && v.strides[vecaxis] == 1 && win_ok && (v.offset % V) == 0;
    for (int d = 0; ok && d < rank; ++d)
      if (d != vecaxis && (v.strides[d] % V) != 0) ok = false;
    leaf_vec[i] = ok;
  }
  if (flat) {
    TPL = 1;
    // one-wave groups for large streams (measured: SwiGLU gate 6.26-6.30 -> 6.47-6.50 TB/s, a
    // 1 GiB copy 6.30 -> 6.42), 256 threads below 2M chunks (a 1M-chunk kernel ran 3 % slower)
    WG = N / std::max(V, 1) >= ((uint64_t)1 << 21) ? 64 : 256;
    if (const char* e = std::getenv("KURUMI_HIP_FLAT_WG")) WG = std::max(64, std::atoi(e) / 64 * 64);
    NC = 1;
    const char* fk = std::getenv("KURUMI_HIP_FLAT_CPT");
    FK = fk ? std::max(1, std::atoi(fk)) : 1;
    return;
  }
  uint64_t chunks = (L + V - 1) / V;
  if (inner > 1) {
    TPL = 1;
    WG = 256;
    GPW = 256;
    NC = (int)chunks;
    return;
  }
  // Chunks of 16 bytes per thread, the line cached in registers. Lines of 4-byte elements take ~8
  // per thread, measured: the f32 [8192, 32000] softmax rows 5.57-5.60 -> 5.74-5.82 TB/s (1024
  // threads per row, from 16 chunks), the f32 [4096, 4096] fused reduce 5.28 -> 5.61 TB/s (128
  // per row); when a full-size output is stored too, ~2 (up to 1024 threads): the f32
  // [8192, 4096] rmsnorm 5.76 -> 5.92 TB/s with 512 threads per row. Lines of 2-byte elements take 256 threads: the bf16 softmax rows (16 chunks each)
  // lose 3-4 % with 512, the bf16 [8192, 4096] rmsnorm rows run at 5.65 TB/s with 32 threads (16
  // chunks each) and 6.79 TB/s with 256 (2 each). Other widths: ~16 chunks per thread.
  // a normalisation (softmax, rmsnorm): a full-size value computed from a line reduction; such
  // regions usually store it, and store-heavy lines want more threads
  bool full_out = false;
  for (size_t i = 0; i < R.nodes.size(); ++i)
    if (full((int)i) && R.nodes[i].level >= 1) full_out = true;
  int target = V == 4 ? (full_out ? 2 : 8) : V == 8 ? (int)std::max<uint64_t>(1, (chunks + 255) / 256) : 16;
  if (const char* e = std::getenv("KURUMI_HIP_LINE_CHUNKS")) target = std::max(1, std::atoi(e));
  uint64_t t = 1;
  while (t < 1024 && t * (uint64_t)target < chunks) t *= 2;
  // few lines: spread each over more threads (down to 2 chunks per thread) until the launch has
  // about 16 waves per CU to hide memory latency with
  while (t < 1024 && lines * t < ((uint64_t)1 << 18) && chunks >= 4 * t) t *= 2;
  TPL = (int)t;
  NC = (int)((chunks + TPL - 1) / TPL);
  // lines of one wave or less share a 256-thread group; a line of several waves is its own group
  // (its cross-wave combine, barriers included, then spans the whole group)
  WG = TPL > 64 ? TPL : 256;
  GPW = WG / TPL;
}

// Phases: level p = 1..P fold reductions of level p; LINE nodes of level p follow.
// FULL outputs of level l are stored in phase l+1 (the final pass P+1 when l == P).
void Gen::schedule() {
  P = 0;
  for (auto& n : R.nodes) P = std::max(P, n.level);
  store_phase.assign(R.nodes.size(), 0);
  for (auto& op : R.outputs) {
    out_slot[op.first] = op.second;
    if (full(op.first) || flat) {
      int l = node(op.first).level;
      store_phase[op.first] = l + 1;
      if (l + 1 > P) has_final = true;
    }
  }
  int nph = P + (has_final ? 1 : 0);
  need.assign(nph + 2, {});
  std::function<void(int, int)> add = [&](int p, int n) {
    if (!full(n) || need[p].count(n)) return;
    need[p].insert(n);
    for (int i : node(n).in) add(p, i);
  };
  for (size_t i = 0; i < R.nodes.size(); ++i) {
    const RNode& n = R.nodes[i];
    if (is_red(n.kind)) add(n.level, n.in[0]);
    if (store_phase[i]) add(store_phase[i], (int)i);
  }
  // cache leaves and reduction inputs that several phases need, when the line fits
  first_phase.assign(R.nodes.size(), 0);
  std::map<int, int> uses;
  for (int p = 1; p <= nph; ++p)
    for (int n : need[p]) {
      uses[n]++;
      if (!first_phase[n]) first_phase[n] = p;
    }
  std::set<int> red_inputs;
  for (auto& n : R.nodes)
    if (is_red(n.kind)) red_inputs.insert(n.in[0]);
  unroll = !flat && NC <= 16;
  if (!flat && NC <= 16) {
    // Register budget: keep at least two work-groups resident per CU (a line kernel's phases
    // are load-bound then ALU/store-bound, so a second line in flight overlaps them). With
    // W waves per group that is W/2 waves per SIMD out of 512 VGPRs, minus ~28 for the rest.
    int waves_per_simd = std::max(1, WG / 128);
    int limit = std::min(256, (512 / waves_per_simd) / 8 * 8);
    min_waves = waves_per_simd;
    if (const char* e = std::getenv("KURUMI_HIP_LINE_WAVES")) min_waves = std::atoi(e);
    int budget = limit - 28;
    if (const char* e = std::getenv("KURUMI_HIP_CACHE_BUDGET")) budget = std::atoi(e);
    auto cost_of = [&](int c) {
      // half-registers per value: 16-bit leaves are cached two to a register
      int per = packed_cache(c) ? 1 : (dt_width(node(c).dtype) == 8 ? 4 : 2);
      return (NC * V * per + 1) / 2;
    };
    // Leaves first: a leaf needed by two phases and not cached is read from HBM twice, while an
    // uncached intermediate only costs ALU to recompute from cached leaves. Then values feeding
    // later reductions (latest level first).
    std::vector<int> leaves_c, inter_c;
    for (auto& kv : uses) {
      if (kv.second < 2) continue;
      if (node(kv.first).kind == RK_LEAF) leaves_c.push_back(kv.first);
      else if (red_inputs.count(kv.first)) inter_c.push_back(kv.first);
    }
    std::sort(inter_c.begin(), inter_c.end(), [&](int x, int y) { return node(x).level > node(y).level; });
    int regs = 0;
    for (int c : leaves_c)
      if (regs + cost_of(c) <= budget) {
        cached.insert(c);
        regs += cost_of(c);
      }
    for (int c : inter_c)
      if (regs + cost_of(c) <= budget) {
        cached.insert(c);
        regs += cost_of(c);
      }
    // a smaller footprint than the budget allows buys more resident waves: ask for them
    if (!std::getenv("KURUMI_HIP_LINE_WAVES")) min_waves = std::max(min_waves, std::min(8, 512 / (regs + 40)));
  }
  // with caches, later phases need fewer recomputations: rebuild need sets
  if (!cached.empty()) {
    need.assign(nph + 2, {});
    std::function<void(int, int)> add2 = [&](int p, int n) {
      if (!full(n) || need[p].count(n)) return;
      need[p].insert(n);
      if (cached.count(n) && first_phase[n] < p) return;
      for (int i : node(n).in) add2(p, i);
    };
    for (size_t i = 0; i < R.nodes.size(); ++i) {
      const RNode& n = R.nodes[i];
      if (is_red(n.kind)) add2(n.level, n.in[0]);
      if (store_phase[i]) add2(store_phase[i], (int)i);
    }
  }
}

// The stored bits of an immediate constant leaf as a value of its storage type.
static std::string imm_expr(const Leaf& l) {
  size_t w = dt_width(l.dtype);
  const char* U = w == 1 ? "u8" : w == 2 ? "u16" : w == 4 ? "u32" : "u64";
  std::ostringstream e;
  e << "__builtin_bit_cast(" << stype(l.dtype) << ", (" << U << ")0x" << std::hex << l.imm_bits[0] << "ull)";
  return e.str();
}

std::string Gen::leaf_base(int li) const {
  const View& v = R.leaves[li].view;
  int vecaxis = flat ? rank - 1 : a;
  std::ostringstream e;
  e << "(" << ix() << ")(" << v.offset << "ll";
  for (int d = 0; d < rank; ++d) {
    if (d == vecaxis || v.strides[d] == 0) continue;
    e << " + (i64)c" << d << " * " << v.strides[d] << "ll";
  }
  e << ")";
  return e.str();
}

// load leaf node ni for the current chunk: c_expr = coordinate of element j=0 along the vector axis
void Gen::emit_leaf_load(int ni, const std::string& c_expr) {
  const RNode& n = node(ni);
  const Leaf& l = R.leaves[n.leaf];
  const View& v = l.view;
  int vecaxis = flat ? rank - 1 : a;
  std::string T = stype(l.dtype), C = ctype(l.dtype);
  std::string P = "p" + std::to_string(slot_param.at(l.slot));
  std::string base = "b" + std::to_string(n.leaf);
  if (l.imm) {
    o << "      " << T << " r" << ni << "[" << V << "];\n";
    o << "      #pragma unroll\n      for (int j = 0; j < " << V << "; ++j) r" << ni << "[j] = " << imm_expr(l) << ";\n";
    emit_leaf_convert(ni);
    return;
  }
  if (bf16_words(ni)) {
    // bf16 pairs stay packed in 32-bit words (the form the cache keeps); each value is its word's
    // low half shifted up or its high half masked
    const bool ntl = flat ? (flat_nt() & 2) != 0 : (nt_mode() & 2) != 0;
    o << "      u32 rw" << ni << "[" << V / 2 << "];\n";
    o << "      { VecT<u32, " << V / 2 << "> raw = " << (ntl ? "vld_nt(" : "*(") << "(const VecT<u32, " << V / 2
      << ">*)((const " << T << "*)" << P << " + (" << ix() << ")(" << base << " + (" << ix() << ")(" << c_expr
      << "))));\n";
    o << "        #pragma unroll\n        for (int jj = 0; jj < " << V / 2 << "; ++jj) rw" << ni << "[jj] = raw.v[jj]; }\n";
    o << "      float f" << ni << "[" << V << "];\n";
    o << "      #pragma unroll\n      for (int jj = 0; jj < " << V / 2 << "; ++jj) { f" << ni
      << "[2 * jj] = __uint_as_float(rw" << ni << "[jj] << 16); f" << ni << "[2 * jj + 1] = __uint_as_float(rw" << ni
      << "[jj] & 0xffff0000u); }\n";
    return;
  }
  // r<ni>: the stored bits (what a leaf cache keeps), f<ni>: the compute values
  o << "      " << T << " r" << ni << "[" << V << "];\n";
  if (leaf_vec[n.leaf] && v.padded()) {
    std::string coord = "((i64)(" + c_expr + "))";
    o << "      if (vb" << n.leaf << " && " << coord << " >= " << v.wlo[vecaxis] << " && " << coord << " < "
      << v.whi[vecaxis] << ") { VecT<" << T << ", " << V << "> raw = *((const VecT<" << T << ", " << V
      << ">*)((const " << T << "*)" << P << " + (" << ix() << ")(" << base << " + (" << ix() << ")(" << c_expr
      << "))));\n";
    o << "        #pragma unroll\n        for (int j = 0; j < " << V << "; ++j) r" << ni << "[j] = raw.v[j];\n";
    o << "      } else {\n        #pragma unroll\n        for (int j = 0; j < " << V << "; ++j) r" << ni << "[j] = ("
      << T << ")0;\n      }\n";
  } else if (leaf_vec[n.leaf]) {
    const bool ntl = flat ? (flat_nt() & 2) != 0 : (nt_mode() & 2) != 0;
    o << "      { VecT<" << T << ", " << V << "> raw = " << (ntl ? "vld_nt(" : "*(") << "(const VecT<" << T << ", " << V
      << ">*)((const " << T << "*)" << P << " + (" << ix() << ")(" << base << " + (" << ix() << ")(" << c_expr
      << "))));\n";
    o << "        #pragma unroll\n        for (int j = 0; j < " << V << "; ++j) r" << ni << "[j] = raw.v[j]; }\n";
  } else {
    int64_t sa = v.strides[vecaxis];
    o << "      #pragma unroll\n      for (int j = 0; j < " << V << "; ++j) {\n";
    std::string coord = "((i64)(" + c_expr + ") + j)";
    std::string off = base + " + (" + ix() + ")(" + coord + " * " + std::to_string(sa) + "ll)";
    std::string load = "((const " + T + "*)" + P + ")[" + off + "]";
    if (v.padded()) {
      std::string inr = "(vb" + std::to_string(n.leaf) + " && " + coord + " >= " + std::to_string(v.wlo[vecaxis]) +
                        " && " + coord + " < " + std::to_string(v.whi[vecaxis]) + ")";
      o << "        r" << ni << "[j] = " << inr << " ? " << load << " : (" << T << ")0;\n";
    } else {
      o << "        r" << ni << "[j] = " << load << ";\n";
    }
    o << "      }\n";
  }
  emit_leaf_convert(ni);
}

void Gen::emit_leaf_convert(int ni) {
  const Leaf& l = R.leaves[node(ni).leaf];
  o << "      " << ctype(l.dtype) << " f" << ni << "[" << V << "];\n";
  o << "      #pragma unroll\n      for (int j = 0; j < " << V << "; ++j) f" << ni << "[j] = "
    << ld(l.dtype, "r" + std::to_string(ni) + "[j]") << ";\n";
}

void Gen::emit_full_node(int ni, int phase, const std::string& c_expr) {
  const RNode& n = node(ni);
  bool from_cache = cached.count(ni) && first_phase[ni] < phase;
  if (from_cache) {
    if (bf16_packed(ni)) {
      // bf16 pairs to f32 without unpacking to 16-bit values: low half << 16, high half masked
      o << "      float f" << ni << "[" << V << "];\n";
      o << "      #pragma unroll\n      for (int jj = 0; jj < " << V / 2 << "; ++jj) { f" << ni
        << "[2 * jj] = __uint_as_float(cache" << ni << "[c][jj] << 16); f" << ni << "[2 * jj + 1] = __uint_as_float(cache"
        << ni << "[c][jj] & 0xffff0000u); }\n";
    } else if (packed_cache(ni)) {
      o << "      " << stype(R.leaves[n.leaf].dtype) << " r" << ni << "[" << V << "];\n";
      o << "      #pragma unroll\n      for (int j = 0; j < " << V << "; ++j) r" << ni << "[j] = (u16)(cache" << ni
        << "[c][j >> 1] >> ((j & 1) * 16));\n";
      emit_leaf_convert(ni);
    } else if (n.kind == RK_LEAF) {
      o << "      " << stype(R.leaves[n.leaf].dtype) << " (&r" << ni << ")[" << V << "] = cache" << ni << "[c];\n";
      emit_leaf_convert(ni);
    } else {
      o << "      " << ctype(n.dtype) << " (&f" << ni << ")[" << V << "] = cache" << ni << "[c];\n";
    }
    return;
  }
  if (n.kind == RK_LEAF) {
    emit_leaf_load(ni, c_expr);
  } else if (n.kind == RK_PADSEL) {
    // zero outside the pad windows; the non-vector axes are tested once, the vector axis per j
    int vecaxis = flat ? rank - 1 : a;
    std::ostringstream cond;
    cond << "true";
    for (int d = 0; d < rank; ++d) {
      if (d == vecaxis) continue;
      if (n.win.wlo[d] > 0) cond << " && (i64)c" << d << " >= " << n.win.wlo[d];
      if (n.win.whi[d] < (int64_t)R.S[d]) cond << " && (i64)c" << d << " < " << n.win.whi[d];
    }
    std::string cj = "((i64)(" + c_expr + ") + j)";
    std::ostringstream condj;
    condj << "pin" << ni;
    if (n.win.wlo[vecaxis] > 0) condj << " && " << cj << " >= " << n.win.wlo[vecaxis];
    if (n.win.whi[vecaxis] < (int64_t)R.S[vecaxis]) condj << " && " << cj << " < " << n.win.whi[vecaxis];
    o << "      const bool pin" << ni << " = " << cond.str() << ";\n";
    o << "      " << ctype(n.dtype) << " f" << ni << "[" << V << "];\n";
    o << "      #pragma unroll\n      for (int j = 0; j < " << V << "; ++j) f" << ni << "[j] = (" << condj.str()
      << ") ? " << val(n.in[0], "j") << " : (" << ctype(n.dtype) << ")0;\n";
  } else if (n.kind == (int)OpKind::Iota || n.kind == (int)OpKind::RandUniform) {
    int vecaxis = flat ? rank - 1 : a;
    o << "      " << ctype(n.dtype) << " f" << ni << "[" << V << "];\n";
    o << "      #pragma unroll\n      for (int j = 0; j < " << V << "; ++j) {\n";
    if (n.kind == (int)OpKind::Iota) {
      std::string coord = ((int)n.axis == vecaxis) ? "((i64)(" + c_expr + ") + j)" : "(i64)c" + std::to_string(n.axis);
      o << "        f" << ni << "[j] = " << cast_expr(DType::I64, n.dtype, coord) << ";\n";
    } else {
      // flat index over S
      std::vector<size_t> rs = row_major_strides(R.S);
      std::ostringstream fi;
      fi << "(u64)0";
      for (int d = 0; d < rank; ++d) {
        if (d == vecaxis) fi << " + ((u64)(" << c_expr << ") + (u64)j) * " << rs[d] << "ull";
        else fi << " + (u64)c" << d << " * " << rs[d] << "ull";
      }
      o << "        f" << ni << "[j] = uniform_f32(threefry2x32((u64)(i64)" << val(n.in[0], "j") << ", " << fi.str()
        << "));\n";
    }
    o << "      }\n";
  } else {
    o << "      " << ctype(n.dtype) << " f" << ni << "[" << V << "];\n";
    std::string e0 = op_expr(ni, "(2 * jj)"), e1 = op_expr(ni, "(2 * jj + 1)");
    const std::string pre = "rbf16(";
    // the whole expression must be one rbf16(...) call: its opening parenthesis closes at the end
    auto wrapped = [&](const std::string& e) {
      if (e.compare(0, pre.size(), pre) != 0 || e.back() != ')') return false;
      int depth = 0;
      for (size_t i = pre.size() - 1; i < e.size(); ++i) {
        if (e[i] == '(') ++depth;
        else if (e[i] == ')' && --depth == 0) return i == e.size() - 1;
      }
      return false;
    };
    if (n.dtype == DType::BF16 && V % 2 == 0 && wrapped(e0) && wrapped(e1)) {
      // bf16 results rounded two at a time (one v_cvt_pk_bf16_f32 per pair)
      e0 = e0.substr(pre.size(), e0.size() - pre.size() - 1);
      e1 = e1.substr(pre.size(), e1.size() - pre.size() - 1);
      o << "      #pragma unroll\n      for (int jj = 0; jj < " << V / 2 << "; ++jj) { float a_ = " << e0
        << "; float b_ = " << e1 << "; rbf16x2(a_, b_); f" << ni << "[2 * jj] = a_; f" << ni << "[2 * jj + 1] = b_; }\n";
    } else {
      o << "      #pragma unroll\n      for (int j = 0; j < " << V << "; ++j) f" << ni << "[j] = " << op_expr(ni, "j")
        << ";\n";
    }
  }
  if (cached.count(ni) && first_phase[ni] == phase) {
    if (bf16_words(ni))
      o << "      #pragma unroll\n      for (int jj = 0; jj < " << V / 2 << "; ++jj) cache" << ni << "[c][jj] = rw" << ni
        << "[jj];\n";
    else if (bf16_packed(ni) && n.kind != RK_LEAF)
      o << "      #pragma unroll\n      for (int jj = 0; jj < " << V / 2 << "; ++jj) cache" << ni
        << "[c][jj] = pack_bf16_exact(f" << ni << "[2 * jj], f" << ni << "[2 * jj + 1]);\n";
    else if (packed_cache(ni))
      o << "      #pragma unroll\n      for (int j = 0; j < " << V / 2 << "; ++j) cache" << ni << "[c][j] = (u32)r" << ni
        << "[2 * j] | ((u32)r" << ni << "[2 * j + 1] << 16);\n";
    else
      o << "      #pragma unroll\n      for (int j = 0; j < " << V << "; ++j) cache" << ni << "[c][j] = "
        << (n.kind == RK_LEAF ? "r" : "f") << ni << "[j];\n";
  }
}

void Gen::emit_line_node(int ni) {
  const RNode& n = node(ni);
  if (n.kind == RK_LEAF) {
    const Leaf& l = R.leaves[n.leaf];
    std::string P = "p" + std::to_string(slot_param.at(l.slot));
    std::string raw = l.imm ? imm_expr(l)
                            : "((const " + std::string(stype(l.dtype)) + "*)" + P + ")[b" + std::to_string(n.leaf) + "]";
    o << "  const " << ctype(n.dtype) << " s" << ni << " = " << ld(l.dtype, raw) << ";\n";
  } else {
    o << "  const " << ctype(n.dtype) << " s" << ni << " = " << op_expr(ni, "0") << ";\n";
  }
  if (needs_line_recip(ni)) o << "  const float s" << ni << "_inv = 1.0f / s" << ni << ";\n";
  auto it = out_slot.find(ni);
  if (it != out_slot.end() && !full(ni) && !flat) {
    o << "  if (lane == 0) ((" << stype(n.dtype) << "*)p" << slot_param.at(it->second) << ")[line] = "
      << st(n.dtype, "s" + std::to_string(ni)) << ";\n";
  }
}

void Gen::emit_red_init(int ni) {
  const RNode& n = node(ni);
  DType in = node(n.in[0]).dtype;
  std::string r = std::to_string(ni);
  if (n.kind == (int)OpKind::ArgReduce) {
    bool mx = n.arg == ArgKind::Max;
    std::string init;
    if (fvalued(in) || in == DType::F64) init = flt_lit(in == DType::F64 ? DType::F64 : DType::F32, mx ? -INFINITY : INFINITY);
    else init = mx ? int_min(in) : int_max(in);
    o << "  " << ctype(in) << " bv" << r << " = " << init << "; " << aix() << " bi" << r << " = " << aix_none()
      << "; bool bn" << r << " = false;\n";
    if (chunk_arg(ni)) {
      // the winning chunk: its first element index and its values (bf16 values two to a word)
      o << "  " << aix() << " bc" << r << " = " << aix_none() << "; ";
      if (chunk_arg_packed(ni)) o << "u32 sw" << r << "[" << V / 2 << "] = {};\n";
      else o << "float sv" << r << "[" << V << "] = {};\n";
    }
    return;
  }
  DType acc = n.dtype;
  std::string A;
  if (fvalued(acc) || in == DType::F32) A = "float";
  else if (acc == DType::F64) A = "double";
  else A = n.kind == (int)OpKind::ReduceMax ? stype(acc) : utype(acc);
  std::string init;
  if (n.kind == (int)OpKind::Sum) init = "(" + A + ")0";
  else if (n.kind == (int)OpKind::Prod) init = "(" + A + ")1";
  else init = (A == "float" || A == "double") ? flt_lit(A == "double" ? DType::F64 : DType::F32, -INFINITY) : int_min(acc);
  o << "  " << A << " acc" << r << " = " << init << ";\n";
}

void Gen::emit_red_update(int ni, const std::string& k_expr, const std::string& j) {
  const RNode& n = node(ni);
  DType in = node(n.in[0]).dtype;
  std::string r = std::to_string(ni);
  std::string v = val(n.in[0], j);
  if (n.kind == (int)OpKind::ArgReduce) {
    bool mx = n.arg == ArgKind::Max;
    std::string cmp = mx ? ">" : "<";
    // A thread visits its elements in increasing k, so within the thread a strict comparison
    // keeps the first index of equal values; NaN never compares true and is skipped. The
    // reference's NaN-at-index-0 rule (the result is 0) is a flag set by the element k == 0.
    std::string k = "((" + aix() + ")(" + k_expr + "))";
    o << "        { " << ctype(in) << " v_ = " << v << "; if (v_ " << cmp << " bv" << r << ") { bv" << r
      << " = v_; bi" << r << " = " << k << "; }";
    if (fvalued(in) || in == DType::F64) o << " if (" << j << " == 0 && " << k << " == 0 && v_ != v_) bn" << r << " = true;";
    o << " }\n";
    return;
  }
  bool fl = fvalued(n.dtype) || n.dtype == DType::F64 || in == DType::F32;
  if (n.kind == (int)OpKind::Sum) {
    if (fl) o << "        acc" << r << " += " << v << ";\n";
    else o << "        acc" << r << " = acc" << r << " + (" << utype(n.dtype) << ")" << v << ";\n";
  } else if (n.kind == (int)OpKind::Prod) {
    if (fl) o << "        acc" << r << " *= " << v << ";\n";
    else o << "        acc" << r << " = acc" << r << " * (" << utype(n.dtype) << ")" << v << ";\n";
  } else {
    if (n.dtype == DType::F64) o << "        acc" << r << " = fmax(acc" << r << ", " << v << ");\n";
    else if (fl) o << "        acc" << r << " = fmaxf(acc" << r << ", " << v << ");\n";
    else o << "        acc" << r << " = (" << v << " > acc" << r << ") ? " << v << " : acc" << r << ";\n";
  }
}

// One chunk of a float ArgReduce (see chunk_arg): the chunk's extreme by maxNum / minNum (NaN
// never wins, as in the per-element rule), a strict comparison with the running best so the first
// chunk holding the best value keeps it, and the reference's NaN-at-index-0 flag from element 0.
void Gen::emit_red_chunk_arg(int ni) {
  const RNode& n = node(ni);
  std::string r = std::to_string(ni);
  const bool mx = n.arg == ArgKind::Max;
  const std::string f = mx ? "fmaxf" : "fminf", cmp = mx ? ">" : "<";
  o << "      { float cm_ = " << val(n.in[0], "0") << ";\n";
  o << "        #pragma unroll\n        for (int j = 1; j < " << V << "; ++j) cm_ = " << f << "(cm_, " << val(n.in[0], "j")
    << ");\n";
  o << "        if (ch == 0u && " << val(n.in[0], "0") << " != " << val(n.in[0], "0") << ") bn" << r << " = true;\n";
  o << "        const bool up_ = cm_ " << cmp << " bv" << r << ";\n";
  o << "        bv" << r << " = up_ ? cm_ : bv" << r << "; bc" << r << " = up_ ? (" << aix() << ")(ch * " << V << "u) : bc" << r
    << ";\n";
  if (chunk_arg_packed(ni))
    o << "        #pragma unroll\n        for (int jj = 0; jj < " << V / 2 << "; ++jj) sw" << r << "[jj] = up_ ? pack_bf16_exact("
      << val(n.in[0], "2 * jj") << ", " << val(n.in[0], "2 * jj + 1") << ") : sw" << r << "[jj];\n";
  else
    o << "        #pragma unroll\n        for (int j = 0; j < " << V << "; ++j) sv" << r << "[j] = up_ ? " << val(n.in[0], "j")
      << " : sv" << r << "[j];\n";
  o << "      }\n";
}

// cross-lane fold of a reduction (butterfly within the wave, LDS across waves)
void Gen::emit_red_finish(int ni, int phase) {
  const RNode& n = node(ni);
  std::string r = std::to_string(ni);
  bool arg = n.kind == (int)OpKind::ArgReduce;
  DType in = node(n.in[0]).dtype;
  auto comb_arg = [&](const std::string& ov, const std::string& oi, const std::string& on) {
    std::string cmp = n.arg == ArgKind::Max ? ">" : "<";
    std::string ok = (fvalued(in) || in == DType::F64) ? "(" + ov + " == " + ov + ") && " : "";
    return "{ if (" + ok + "(" + ov + " " + cmp + " bv" + r + " || (" + ov + " == bv" + r + " && " + oi + " < bi" + r +
           "))) { bv" + r + " = " + ov + "; bi" + r + " = " + oi + "; } bn" + r + " = bn" + r + " || " + on + "; }";
  };
  auto comb = [&](const std::string& ov) {
    if (n.kind == (int)OpKind::Sum) return "acc" + r + " = acc" + r + " + " + ov + ";";
    if (n.kind == (int)OpKind::Prod) return "acc" + r + " = acc" + r + " * " + ov + ";";
    if (n.dtype == DType::F64) return "acc" + r + " = fmax(acc" + r + ", " + ov + ");";
    if (fvalued(n.dtype) || in == DType::F32) return "acc" + r + " = fmaxf(acc" + r + ", " + ov + ");";
    return "acc" + r + " = (" + ov + " > acc" + r + ") ? " + ov + " : acc" + r + ";";
  };
  if (chunk_arg(ni)) {
    // the index of the first element of the winning chunk equal to the best value
    o << "  if (bc" << r << " != " << aix_none() << ") {\n    " << aix() << " bj_ = " << V - 1 << ";\n";
    if (chunk_arg_packed(ni))
      o << "    #pragma unroll\n    for (int j = " << V - 1 << "; j >= 0; --j) { const float v_ = __uint_as_float((j & 1) ? (sw" << r
        << "[j >> 1] & 0xffff0000u) : (sw" << r << "[j >> 1] << 16)); if (v_ == bv" << r << ") bj_ = j; }\n";
    else
      o << "    #pragma unroll\n    for (int j = " << V - 1 << "; j >= 0; --j) if (sv" << r << "[j] == bv" << r << ") bj_ = j;\n";
    o << "    bi" << r << " = bc" << r << " + bj_;\n  }\n";
  }
  int wl = std::min(TPL, 64);
  const bool fsum = n.kind == (int)OpKind::Sum && (fvalued(n.dtype) || in == DType::F32);
  const bool fmax = n.kind == (int)OpKind::ReduceMax && (fvalued(n.dtype) || in == DType::F32);
  static const bool no_dpp = std::getenv("KURUMI_HIP_NO_DPP") != nullptr;
  if (!arg && wl == 64 && (fsum || fmax) && !no_dpp) {
    o << "  acc" << r << " = " << (fsum ? "wave_sum(" : "wave_max(") << "acc" << r << ");\n";
    wl = 1;  // folded; the loop below does nothing
  }
  for (int m = wl / 2; m >= 1; m /= 2) {
    if (arg)
      o << "  { " << ctype(in) << " ov = shx(bv" << r << ", " << m << "); " << aix() << " oi = shx(bi" << r << ", " << m
        << "); bool on = shx(bn" << r << ", " << m << "); " << comb_arg("ov", "oi", "on") << " }\n";
    else
      o << "  { auto ov = shx(acc" << r << ", " << m << "); " << comb("ov") << " }\n";
  }
  if (TPL > 64) {
    if (GPW != 1) throw Error("codegen: a multi-wave line must be its own work-group");
    int W = TPL / 64;
    std::string tag = std::to_string(phase) + "_" + r;
    if (arg) {
      o << "  __shared__ " << ctype(in) << " lv" << tag << "[" << W << "]; __shared__ " << aix() << " li" << tag << "[" << W
        << "]; __shared__ bool ln" << tag << "[" << W << "];\n";
      o << "  if ((threadIdx.x & 63) == 0) { lv" << tag << "[threadIdx.x >> 6] = bv" << r << "; li" << tag
        << "[threadIdx.x >> 6] = bi" << r << "; ln" << tag << "[threadIdx.x >> 6] = bn" << r << "; }\n";
      o << "  __syncthreads();\n";
      o << "  bv" << r << " = lv" << tag << "[0]; bi" << r << " = li" << tag << "[0]; bn" << r << " = ln" << tag << "[0];\n";
      o << "  for (int w = 1; w < " << W << "; ++w) { " << ctype(in) << " ov = lv" << tag << "[w]; " << aix() << " oi = li" << tag
        << "[w]; bool on = ln" << tag << "[w]; " << comb_arg("ov", "oi", "on") << " }\n";
    } else {
      o << "  __shared__ decltype(acc" << r << ") lr" << tag << "[" << W << "];\n";
      o << "  if ((threadIdx.x & 63) == 0) lr" << tag << "[threadIdx.x >> 6] = acc" << r << ";\n";
      o << "  __syncthreads();\n";
      o << "  acc" << r << " = lr" << tag << "[0];\n";
      o << "  for (int w = 1; w < " << W << "; ++w) { auto ov = lr" << tag << "[w]; " << comb("ov") << " }\n";
    }
  }
  // final value
  if (arg) {
    o << "  const i64 s" << r << " = (bn" << r << " || bi" << r << " == " << aix_none() << ") ? 0ll : (i64)bi" << r
      << ";\n";
  } else {
    std::string v = "acc" + r;
    if (dt_is_int(n.dtype)) v = std::string("(") + stype(n.dtype) + ")" + v;
    else v = rnd(n.dtype, v);
    o << "  const " << ctype(n.dtype) << " s" << r << " = " << v << ";\n";
    if (needs_line_recip(ni)) o << "  const float s" << r << "_inv = 1.0f / s" << r << ";\n";
  }
  auto it = out_slot.find(ni);
  if (it != out_slot.end()) {
    o << "  if (lane == 0) ((" << stype(n.dtype) << "*)p" << slot_param.at(it->second) << ")[line] = "
      << st(n.dtype, "s" + r) << ";\n";
  }
}

std::string Gen::generate(RegionCode* rc) {
  plan_layout();
  schedule();
  std::ostringstream nm;
  // placeholder entry; the final name carries the iteration shape and a hash of the body so
  // that profiles can tell kernels apart (one name per distinct generated kernel)
  nm << "ku_" << (flat ? "ew" : "line");
  for (size_t d = 0; d < R.S.size(); ++d) nm << (d ? "x" : "_") << R.S[d];
  std::string entry = "KU_ENTRY_PLACEHOLDER";
  std::string prefix = nm.str();
  for (auto& l : R.leaves) param(l.slot);
  for (auto& op : R.outputs) param(op.second);
  o << kDevicePrelude;
  o << "extern \"C\" __global__ void __launch_bounds__(" << WG << ") ";
  // line kernels: ask for the occupancy the cache budget was sized for (two groups per CU)
  if (!flat && min_waves > 1) o << "__attribute__((amdgpu_waves_per_eu(" << min_waves << "))) ";
  o << entry << "(";
  for (size_t i = 0; i < param_slots.size(); ++i) o << (i ? ", " : "") << "void* __restrict__ p" << i;
  o << ") {\n";
  int vecaxis = flat ? rank - 1 : a;
  std::vector<int> lines_leaves;
  if (flat) {
    // FK chunks per thread, each a block-wide coalesced stripe, unrolled so their loads are in
    // flight together
    uint64_t chunks = N / V;
    o << "  #pragma unroll\n  for (int kk = 0; kk < " << FK << "; ++kk) {\n";
    o << "  const u64 chunk = ((u64)blockIdx.x * " << FK << "ull + kk) * " << WG << "ull + threadIdx.x;\n";
    o << "  if (chunk < " << chunks << "ull) {\n";
    o << "  const int lane = 0; (void)lane;\n";
    o << "  " << ix() << " t = (" << ix() << ")(chunk * " << V << "ull);\n";
    for (int d = rank - 1; d >= 0; --d) {
      o << "  const " << ix() << " c" << d << " = t % " << R.S[d] << "u; t /= " << R.S[d] << "u;\n";
    }
    o << "  (void)t;\n";
  } else {
    o << "  const u32 lane = threadIdx.x % " << TPL << "u;\n";
    o << "  const u64 line = (u64)blockIdx.x * " << GPW << "ull + threadIdx.x / " << TPL << "u;\n";
    if ((uint64_t)GPW * (((lines + GPW - 1) / GPW)) != lines) o << "  if (line >= " << lines << "ull) return;\n";
    o << "  " << ix() << " t = (" << ix() << ")line;\n";
    for (int d = rank - 1; d >= 0; --d) {
      if (d == a) continue;
      o << "  const " << ix() << " c" << d << " = t % " << R.S[d] << "u; t /= " << R.S[d] << "u;\n";
    }
    o << "  (void)t;\n";
  }
  // leaf bases (+ padding validity on the non-vector axes)
  for (size_t li = 0; li < R.leaves.size(); ++li) {
    // b<leaf> is the element index modulo the index width: a padded view's offset may lie before
    // the buffer, so the vector-axis term is always added in the index type before the pointer
    o << "  const " << ix() << " b" << li << " = " << leaf_base((int)li) << ";\n";
    const View& v = R.leaves[li].view;
    if (v.padded()) {
      o << "  const bool vb" << li << " = true";
      for (int d = 0; d < rank; ++d) {
        if (d == vecaxis) continue;
        if (v.wlo[d] > 0) o << " && (i64)c" << d << " >= " << v.wlo[d];
        if (v.whi[d] < (int64_t)v.shape[d]) o << " && (i64)c" << d << " < " << v.whi[d];
      }
      o << ";\n";
    }
  }
  if (flat) {
    // single pass over V elements
    std::string cexpr = "c" + std::to_string(rank - 1);
    std::set<int> needed;
    std::function<void(int)> add = [&](int n) {
      if (needed.count(n)) return;
      needed.insert(n);
      for (int i : node(n).in) add(i);
    };
    for (auto& op : R.outputs) add(op.first);
    o << "  {\n";
    for (size_t i = 0; i < R.nodes.size(); ++i)
      if (needed.count((int)i)) emit_full_node((int)i, 1, cexpr);
    for (auto& op : R.outputs) {
      const RNode& n = node(op.first);
      std::string T = stype(n.dtype);
      std::string P = "p" + std::to_string(slot_param.at(op.second));
      if (V > 1 && n.dtype == DType::BF16 && V % 2 == 0 && n.kind != RK_LEAF) {
        // every bf16 op result is already bf16-exact: pack pairs with one v_perm each
        o << "    { VecT<u32, " << V / 2 << "> w;\n      #pragma unroll\n      for (int jj = 0; jj < " << V / 2
          << "; ++jj) w.v[jj] = pack_bf16_exact(f" << op.first << "[2 * jj], f" << op.first << "[2 * jj + 1]);\n"
          << "      " << (flat_nt() & 1 ? "vst_nt(" : "*(") << "(VecT<u32, " << V / 2 << ">*)((" << T << "*)" << P
          << " + chunk * " << V << "ull)" << (flat_nt() & 1 ? ", w); }\n" : ") = w; }\n");
      } else if (V > 1) {
        o << "    { VecT<" << T << ", " << V << "> w;\n      #pragma unroll\n      for (int j = 0; j < " << V
          << "; ++j) w.v[j] = " << st(n.dtype, "f" + std::to_string(op.first) + "[j]") << ";\n      "
          << (flat_nt() & 1 ? "vst_nt(" : "*(") << "(VecT<" << T << ", " << V << ">*)((" << T << "*)" << P << " + chunk * "
          << V << "ull)" << (flat_nt() & 1 ? ", w); }\n" : ") = w; }\n");
      } else {
        o << "    ((" << T << "*)" << P << ")[chunk] = " << st(n.dtype, "f" + std::to_string(op.first) + "[0]") << ";\n";
      }
    }
    o << "  }\n  }\n  }\n}\n";
    rc->grid = (unsigned)((N / (uint64_t)V + (uint64_t)WG * FK - 1) / ((uint64_t)WG * FK));
    rc->block = WG;
    rc->arg_slots = param_slots;
    return finish(prefix, rc);
  }
  // ---- line kernel ----
  // caches
  for (int c : cached) {
    const RNode& cn = node(c);
    if (packed_cache(c)) o << "  u32 cache" << c << "[" << NC << "][" << V / 2 << "];\n";
    else o << "  " << (cn.kind == RK_LEAF ? stype(R.leaves[cn.leaf].dtype) : ctype(cn.dtype)) << " cache" << c << "["
           << NC << "][" << V << "];\n";
  }
  // line-level (level 0) LINE nodes
  for (size_t i = 0; i < R.nodes.size(); ++i)
    if (!full((int)i) && node((int)i).level == 0 && !is_red(node((int)i).kind)) emit_line_node((int)i);
  std::vector<size_t> rs = row_major_strides(R.S);
  int nph = P + (has_final ? 1 : 0);
  for (int p = 1; p <= nph; ++p) {
    std::vector<int> reds;
    for (size_t i = 0; i < R.nodes.size(); ++i)
      if (is_red(node((int)i).kind) && node((int)i).level == p) reds.push_back((int)i);
    for (int r : reds) emit_red_init(r);
    // chunk loop
    if (unroll) o << "  #pragma unroll\n";
    else o << "  #pragma unroll 2\n";
    o << "  for (int c = 0; c < " << NC << "; ++c) {\n";
    o << "    const u32 ch = (u32)c * " << TPL << "u + lane;\n";
    bool guard = (uint64_t)NC * TPL * V != L;
    if (guard) o << "    if ((u64)ch * " << V << "ull < " << L << "ull) {\n";
    else o << "    {\n";
    std::string cexpr = "ch * " + std::to_string(V) + "u";
    for (size_t i = 0; i < R.nodes.size(); ++i)
      if (need[p].count((int)i)) emit_full_node((int)i, p, cexpr);
    for (int r : reds) {
      if (chunk_arg(r)) {
        emit_red_chunk_arg(r);
        continue;
      }
      o << "      #pragma unroll\n      for (int j = 0; j < " << V << "; ++j) {\n";
      emit_red_update(r, "ch * " + std::to_string(V) + "u + j", "j");
      o << "      }\n";
    }
    // FULL outputs stored in this phase
    for (auto& op : R.outputs) {
      if (!full(op.first) || store_phase[op.first] != p) continue;
      const RNode& n = node(op.first);
      std::string T = stype(n.dtype);
      std::string Pp = "p" + std::to_string(slot_param.at(op.second));
      // output offset: row-major over S
      std::ostringstream ob;
      ob << "(" << ix() << ")(0";
      for (int d = 0; d < rank; ++d)
        if (d != a) ob << " + (" << ix() << ")c" << d << " * " << rs[d] << "u";
      ob << ")";
      if (V > 1 && rs[a] == 1) {
        const bool nts = nt_mode() & 1;
        if (n.dtype == DType::BF16 && V % 2 == 0 && full(op.first)) {
          // every bf16 value is carried bf16-exact in f32: its pattern is the upper half
          o << "      { VecT<u32, " << V / 2 << "> w;\n        #pragma unroll\n        for (int jj = 0; jj < " << V / 2
            << "; ++jj) w.v[jj] = pack_bf16_exact(" << val(op.first, "2 * jj") << ", " << val(op.first, "2 * jj + 1")
            << ");\n        " << (nts ? "vst_nt(" : "*(") << "(VecT<u32, " << V / 2 << ">*)((" << T << "*)" << Pp << " + "
            << ob.str() << " + (" << ix() << ")(" << cexpr << "))" << (nts ? ", w); }\n" : ") = w; }\n");
        } else {
          o << "      { VecT<" << T << ", " << V << "> w;\n        #pragma unroll\n        for (int j = 0; j < " << V
            << "; ++j) w.v[j] = " << st(n.dtype, val(op.first, "j")) << ";\n        " << (nts ? "vst_nt(" : "*(")
            << "(VecT<" << T << ", " << V << ">*)((" << T << "*)" << Pp << " + " << ob.str() << " + (" << ix() << ")("
            << cexpr << "))" << (nts ? ", w); }\n" : ") = w; }\n");
        }
      } else {
        o << "      #pragma unroll\n      for (int j = 0; j < " << V << "; ++j) ((" << T << "*)" << Pp << ")["
          << ob.str() << " + ((" << ix() << ")(" << cexpr << ") + j) * " << rs[a] << "u] = "
          << st(n.dtype, val(op.first, "j")) << ";\n";
      }
    }
    o << "    }\n  }\n";
    for (int r : reds) emit_red_finish(r, p);
    for (size_t i = 0; i < R.nodes.size(); ++i)
      if (!full((int)i) && node((int)i).level == p && !is_red(node((int)i).kind)) emit_line_node((int)i);
  }
  o << "}\n";
  rc->grid = (unsigned)((lines + GPW - 1) / GPW);
  rc->block = WG;
  rc->arg_slots = param_slots;
  return finish(prefix, rc);
}

}  // namespace

RegionCode gen_region(const Region& r, const std::vector<Slot>& slots, int index) {
  Gen g(r, slots, index);
  RegionCode rc;
  rc.src = g.generate(&rc);
  return rc;
}

}  // namespace ku::hipbk
