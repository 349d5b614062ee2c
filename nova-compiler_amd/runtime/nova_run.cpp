// libnova_run: MLIR-free planner and executor for Nova programs in the op
// surface of this path (C ABI in include/nova_run.h).
//
// Three stages:
//   parse   -- a small reader for the textual IR nova-opt consumes: func.func
//              signatures, one op per statement (lines joined while brackets
//              are open), nova / linalg / tensor / arith / bufferization ops
//              of the subset, tensor and memref types with static shapes.
//              Result types of nova ops are inferred as the reference's
//              inferReturnTypes do (NovaOps.cpp:1116-1285 matmul, 2032-2053
//              layer_norm, 2075-2103 linear, 1648-1677 sce).
//   plan    -- each value gets a physical view (buffer, shape, strides,
//              stored dtype).  nova.transpose of the last two dims is a view;
//              a widening nova.cast (bf16/f16 -> f32, exact) keeps the stored
//              dtype, so the GEMM that consumes it reads the narrow operand
//              directly (the config-2/3 forms nova.cast -> nova.matmul /
//              nova.linear); a nova.gelu and a narrowing nova.cast on a GEMM
//              result with no other use fold into the GEMM epilogue
//              (FuseMatmulBias.cpp:95-199 puts the bias there already).  Every
//              remaining op maps to one libnova_hip entry point.
//   execute -- device buffers for every planned buffer, host->device copies
//              of the arguments, the launches on the calling thread's stream,
//              one synchronisation, device->host copies of the results.
#include <errno.h>
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <memory>
#include <mutex>
#include <set>
#include <string>
#include <vector>

#include "../../include/nova_forms.h"
#include "../../include/nova_hip.h"
#include "../../include/nova_run.h"

namespace {

thread_local char t_err[1024] = {0};

int32_t fail(int32_t code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(t_err, sizeof(t_err), fmt, ap);
  va_end(ap);
  return code;
}

enum { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2, DT_I32 = 3, DT_I64 = 4, DT_I16 = 5 };
const char *dt_name(int dt) {
  static const char *n[] = {"f32", "bf16", "f16", "i32", "i64", "i16"};
  return dt >= 0 && dt <= 5 ? n[dt] : "?";
}
int dt_size(int dt) { return dt == DT_F32 || dt == DT_I32 ? 4 : dt == DT_I64 ? 8 : 2; }
bool is_index_dt(int dt) { return dt == DT_I32 || dt == DT_I64 || dt == DT_I16; }

struct Type {
  std::vector<int64_t> shape;
  int dt = -1;
  bool memref = false;
  int64_t numel() const {
    int64_t n = 1;
    for (int64_t d : shape) n *= d;
    return n;
  }
};

struct Op {
  std::string name;
  std::vector<std::string> results;
  std::vector<std::string> operands;
  std::vector<Type> operand_types;
  std::vector<Type> result_types;
  std::map<std::string, std::string> attrs;
  std::string literal;  // arith.constant value
  int line = 0;
};

struct Func {
  std::string name;
  std::vector<std::string> arg_names;
  std::vector<Type> arg_types;
  std::vector<Op> ops;
  std::vector<std::string> rets;
  std::vector<Type> ret_types;
};

// ---- text helpers ----------------------------------------------------------
std::string trim(const std::string &s) {
  size_t a = 0, b = s.size();
  while (a < b && isspace((unsigned char)s[a])) ++a;
  while (b > a && isspace((unsigned char)s[b - 1])) --b;
  return s.substr(a, b - a);
}

// Split at top-level occurrences of `sep` (outside (), <>, [], {}).
std::vector<std::string> split_top(const std::string &s, char sep) {
  std::vector<std::string> out;
  int depth = 0;
  size_t start = 0;
  for (size_t i = 0; i < s.size(); ++i) {
    const char c = s[i];
    if (c == '(' || c == '<' || c == '[' || c == '{') ++depth;
    else if (c == ')' || c == '>' || c == ']' || c == '}') --depth;
    else if (c == sep && depth == 0) {
      out.push_back(trim(s.substr(start, i - start)));
      start = i + 1;
    }
  }
  out.push_back(trim(s.substr(start)));
  if (out.size() == 1 && out[0].empty()) out.clear();
  return out;
}

// Index of the first top-level `c`, or npos.
size_t find_top(const std::string &s, char c, size_t from = 0) {
  int depth = 0;
  for (size_t i = from; i < s.size(); ++i) {
    const char x = s[i];
    if (x == c && depth == 0) return i;
    if (x == '(' || x == '<' || x == '[' || x == '{') ++depth;
    else if (x == ')' || x == '>' || x == ']' || x == '}') --depth;
  }
  return std::string::npos;
}

// Matching close bracket for the open one at s[i].
size_t match_close(const std::string &s, size_t i) {
  const char open = s[i];
  const char close = open == '(' ? ')' : open == '{' ? '}' : open == '[' ? ']' : '>';
  int depth = 0;
  for (size_t j = i; j < s.size(); ++j) {
    if (s[j] == open) ++depth;
    else if (s[j] == close && --depth == 0) return j;
  }
  return std::string::npos;
}

bool parse_type(const std::string &s_in, Type &t) {
  const std::string s = trim(s_in);
  size_t lt = s.find('<');
  if (lt == std::string::npos) return false;
  const std::string kind = trim(s.substr(0, lt));
  if (kind != "tensor" && kind != "memref") return false;
  t.memref = kind == "memref";
  const size_t gt = match_close(s, lt);
  if (gt == std::string::npos) return false;
  std::string body = s.substr(lt + 1, gt - lt - 1);
  // memref<...xf32, 1>: drop a memory space / layout after the first comma
  const size_t comma = find_top(body, ',');
  if (comma != std::string::npos) body = body.substr(0, comma);
  body = trim(body);
  t.shape.clear();
  size_t pos = 0;
  while (true) {
    const size_t x = body.find('x', pos);
    const std::string tok = body.substr(pos, x == std::string::npos ? std::string::npos : x - pos);
    if (!tok.empty() && isdigit((unsigned char)tok[0]) && x != std::string::npos) {
      // Every size product below is plain int64 arithmetic: a dimension
      // past 2^40 (or digits that do not parse whole) and an element count
      // past 2^50 are refused here, so no byte count can overflow.
      errno = 0;
      char *end = nullptr;
      const long long d = strtoll(tok.c_str(), &end, 10);
      if (errno != 0 || *end != '\0' || d > (1LL << 40)) return false;
      int64_t n = d;
      for (int64_t e : t.shape)
        if (e != 0 && n > (int64_t(1) << 50) / e) return false;
        else n *= e;
      if (n > (int64_t(1) << 50)) return false;
      t.shape.push_back(d);
      pos = x + 1;
      continue;
    }
    const std::string el = trim(body.substr(pos));
    if (el == "f32") t.dt = DT_F32;
    else if (el == "bf16") t.dt = DT_BF16;
    else if (el == "f16") t.dt = DT_F16;
    else if (el == "i32") t.dt = DT_I32;
    else if (el == "i64") t.dt = DT_I64;
    else if (el == "i16") t.dt = DT_I16;
    else return false;
    return true;
  }
}

// Strip `//` comments.
std::string strip_comments(const std::string &text) {
  std::string out;
  size_t i = 0;
  while (i < text.size()) {
    const size_t nl = text.find('\n', i);
    std::string line = text.substr(i, nl == std::string::npos ? std::string::npos : nl - i);
    const size_t c = line.find("//");
    if (c != std::string::npos) line = line.substr(0, c);
    out += line;
    out += '\n';
    if (nl == std::string::npos) break;
    i = nl + 1;
  }
  return out;
}

int line_of(const std::string &text, size_t pos) {
  int n = 1;
  for (size_t i = 0; i < pos && i < text.size(); ++i) n += text[i] == '\n';
  return n;
}

// ---- op parsing --------------------------------------------------------------
// Operand names (%x) in a comma list, skipping keyword pairs and attr dicts.
std::vector<std::string> operand_names(const std::string &s) {
  std::vector<std::string> out;
  for (const std::string &part : split_top(s, ',')) {
    std::string p = trim(part);
    if (!p.empty() && p[0] == '%') {
      size_t e = 1;
      while (e < p.size() && (isalnum((unsigned char)p[e]) || p[e] == '_' || p[e] == '#')) ++e;
      out.push_back(p.substr(0, e));
    }
  }
  return out;
}

void parse_attr_dict(const std::string &s, std::map<std::string, std::string> &attrs) {
  const size_t lb = s.find('{');
  if (lb == std::string::npos) return;
  const size_t rb = match_close(s, lb);
  if (rb == std::string::npos) return;
  for (const std::string &kv : split_top(s.substr(lb + 1, rb - lb - 1), ',')) {
    const size_t eq = kv.find('=');
    if (eq == std::string::npos) continue;
    std::string v = trim(kv.substr(eq + 1));
    const size_t colon = find_top(v, ':');
    if (colon != std::string::npos) v = trim(v.substr(0, colon));
    attrs[trim(kv.substr(0, eq))] = v;
  }
}

// `ins(%a, %b : t1, t2)` -> names and types.
bool parse_ins_outs(const std::string &s, const char *kw, std::vector<std::string> &names,
                    std::vector<Type> &types) {
  const size_t k = s.find(kw);
  if (k == std::string::npos) return false;
  const size_t lp = s.find('(', k);
  const size_t rp = lp == std::string::npos ? lp : match_close(s, lp);
  if (rp == std::string::npos) return false;
  const std::string in = s.substr(lp + 1, rp - lp - 1);
  const size_t colon = find_top(in, ':');
  if (colon == std::string::npos) return false;
  names = operand_names(in.substr(0, colon));
  for (const std::string &ts : split_top(in.substr(colon + 1), ',')) {
    Type t;
    if (parse_type(ts, t)) types.push_back(t);
    else if (trim(ts) == "f32" || trim(ts) == "bf16" || trim(ts) == "f16") {
      t.dt = trim(ts) == "f32" ? DT_F32 : trim(ts) == "bf16" ? DT_BF16 : DT_F16;
      types.push_back(t);  // scalar (rank 0)
    } else {
      return false;
    }
  }
  return names.size() == types.size();
}

int32_t parse_op(const std::string &stmt, int line, Op &op) {
  op.line = line;
  std::string rest = stmt;
  const size_t eq = find_top(stmt, '=');
  if (eq != std::string::npos && stmt[0] == '%') {
    for (const std::string &r : split_top(stmt.substr(0, eq), ',')) {
      const size_t colon = r.find(':');
      if (colon != std::string::npos) {  // %r:3
        const std::string base = trim(r.substr(0, colon));
        const int n = atoi(r.c_str() + colon + 1);
        for (int i = 0; i < n; ++i) op.results.push_back(base + "#" + std::to_string(i));
      } else {
        op.results.push_back(trim(r));
      }
    }
    rest = trim(stmt.substr(eq + 1));
  }
  size_t sp = 0;
  while (sp < rest.size() && !isspace((unsigned char)rest[sp]) && rest[sp] != '(') ++sp;
  op.name = rest.substr(0, sp);
  const std::string body = trim(rest.substr(sp));

  if (op.name == "linalg.matmul" || op.name == "linalg.batch_matmul" || op.name == "linalg.fill") {
    std::vector<std::string> in, out;
    std::vector<Type> tin, tout;
    if (!parse_ins_outs(body, "ins", in, tin) || !parse_ins_outs(body, "outs", out, tout))
      return fail(NOVA_HIP_EINVAL, "line %d: cannot read ins/outs of %s", line, op.name.c_str());
    op.operands = in;
    op.operand_types = tin;
    op.operands.insert(op.operands.end(), out.begin(), out.end());
    op.operand_types.insert(op.operand_types.end(), tout.begin(), tout.end());
    op.result_types = tout;
    return NOVA_HIP_SUCCESS;
  }
  if (op.name == "tensor.empty") {
    Type t;
    const size_t colon = find_top(body, ':');
    if (colon == std::string::npos || !parse_type(body.substr(colon + 1), t))
      return fail(NOVA_HIP_EINVAL, "line %d: cannot read tensor.empty type", line);
    op.result_types.push_back(t);
    return NOVA_HIP_SUCCESS;
  }
  if (op.name == "arith.constant") {
    const size_t colon = find_top(body, ':');
    op.literal = trim(body.substr(0, colon));
    return NOVA_HIP_SUCCESS;
  }
  if (op.name == "bufferization.to_tensor") {
    // %arg restrict : memref<...> to tensor<...>
    const size_t colon = find_top(body, ':');
    op.operands = operand_names(body.substr(0, colon));
    const std::string ts = body.substr(colon + 1);
    const size_t to = ts.rfind(" to ");
    Type t;
    if (to == std::string::npos || !parse_type(ts.substr(to + 4), t))
      return fail(NOVA_HIP_EINVAL, "line %d: cannot read bufferization.to_tensor", line);
    op.result_types.push_back(t);
    return NOVA_HIP_SUCCESS;
  }
  if (op.name == "bufferization.materialize_in_destination") {
    // %v in writable %arg : (tensor, memref) -> ()
    const size_t colon = find_top(body, ':');
    std::string head = body.substr(0, colon);
    const size_t in = head.find(" in ");
    if (in == std::string::npos)
      return fail(NOVA_HIP_EINVAL, "line %d: cannot read materialize_in_destination", line);
    op.operands = operand_names(head.substr(0, in));
    std::string dst = trim(head.substr(in + 4));
    if (dst.compare(0, 8, "writable") == 0) dst = trim(dst.substr(8));
    const std::vector<std::string> d = operand_names(dst);
    op.operands.insert(op.operands.end(), d.begin(), d.end());
    return NOVA_HIP_SUCCESS;
  }
  if (op.name.compare(0, 5, "nova.") == 0) {
    const size_t colon = find_top(body, ':');
    if (colon == std::string::npos)
      return fail(NOVA_HIP_EINVAL, "line %d: %s has no type list", line, op.name.c_str());
    std::string head = body.substr(0, colon), tail = body.substr(colon + 1);
    parse_attr_dict(head, op.attrs);
    // keyword attributes written before any attr-dict: nova.transpose's
    // `axes1 = -1 axes2 = -2`, nova.scatter_add's `axis = 0`, nova.reduce's
    // `dimension = [0] keepdims = true`
    for (const char *kw : {"axes1", "axes2", "axis", "keepdims", "dimension"}) {
      const size_t lb0 = head.find('{');
      size_t k = head.find(kw);
      while (k != std::string::npos && k > 0 && (isalnum((unsigned char)head[k - 1]) || head[k - 1] == '_'))
        k = head.find(kw, k + 1);
      if (k == std::string::npos || (lb0 != std::string::npos && k > lb0)) continue;
      const size_t eqk = head.find('=', k);
      if (eqk == std::string::npos) continue;
      std::string v = trim(head.substr(eqk + 1));
      if (!v.empty() && v[0] == '[') {
        v = v.substr(0, match_close(v, 0) + 1);
      } else {
        size_t e = 0;
        while (e < v.size() && (isalnum((unsigned char)v[e]) || v[e] == '-' || v[e] == '_')) ++e;
        v = v.substr(0, e);
      }
      if (strcmp(kw, "axes1") == 0 || strcmp(kw, "axes2") == 0)
        v = std::to_string(strtol(v.c_str(), nullptr, 10));
      op.attrs[kw] = v;
    }
    const size_t lb = head.find('{');
    std::string opnd = lb == std::string::npos ? head : head.substr(0, lb);
    // the keyword part is not an operand list
    for (const char *kw : {" dimension", " keepdims", " ignore_nan", " axis"}) {
      const size_t k = opnd.find(kw);
      if (k != std::string::npos) opnd = opnd.substr(0, k);
    }
    if (op.name == "nova.gather") {
      // `%table [%indices]`
      const size_t lsq = opnd.find('[');
      const size_t rsq = lsq == std::string::npos ? lsq : match_close(opnd, lsq);
      if (rsq == std::string::npos)
        return fail(NOVA_HIP_EINVAL, "line %d: nova.gather needs `%%table [%%indices]`", line);
      op.operands = operand_names(opnd.substr(0, lsq));
      for (const std::string &n : operand_names(opnd.substr(lsq + 1, rsq - lsq - 1)))
        op.operands.push_back(n);
    } else {
      op.operands = operand_names(opnd);
    }
    const size_t arrow = find_top(tail, '-');
    std::string res_t;
    if (arrow != std::string::npos && arrow + 1 < tail.size() && tail[arrow + 1] == '>') {
      res_t = tail.substr(arrow + 2);
      tail = tail.substr(0, arrow);
    }
    for (const std::string &ts : split_top(tail, ',')) {
      Type t;
      if (!parse_type(ts, t))
        return fail(NOVA_HIP_EINVAL, "line %d: unsupported type '%s' (static tensor shapes of f32/bf16/f16/i32/i64 only)",
                    line, ts.c_str());
      op.operand_types.push_back(t);
    }
    if (!res_t.empty()) {
      Type t;
      if (!parse_type(res_t, t)) return fail(NOVA_HIP_EINVAL, "line %d: bad result type", line);
      op.result_types.push_back(t);
    }
    if (op.name == "nova.constant" && op.operands.empty() && op.operand_types.size() == 1 &&
        op.result_types.empty()) {
      op.result_types = op.operand_types;  // `nova.constant {value = ...} : type`
      op.operand_types.clear();
    }
    if (op.operand_types.size() != op.operands.size())
      return fail(NOVA_HIP_EINVAL, "line %d: %s lists %zu operands and %zu types", line,
                  op.name.c_str(), op.operands.size(), op.operand_types.size());
    return NOVA_HIP_SUCCESS;
  }
  return fail(NOVA_HIP_EINVAL, "line %d: op '%s' is not part of this path's op surface", line,
              op.name.c_str());
}

// Reduced dims of a nova.reduce (`dimension = [..]`, all dims when absent),
// normalised to [0, rank).
std::vector<int> reduce_dims(const Op &op, int rank) {
  std::vector<int> dims;
  auto it = op.attrs.find("dimension");
  if (it == op.attrs.end()) {
    for (int i = 0; i < rank; ++i) dims.push_back(i);
    return dims;
  }
  std::string v = it->second;
  if (!v.empty() && v[0] == '[') v = v.substr(1, v.size() - 2);
  for (const std::string &t : split_top(v, ',')) {
    int d = atoi(t.c_str());
    if (d < 0) d += rank;
    dims.push_back(d);
  }
  return dims;
}

// ---- result type inference (the reference's inferReturnTypes) -------------------
int32_t infer(Op &op) {
  auto &T = op.operand_types;
  auto need = [&](size_t n) {
    return T.size() == n ? NOVA_HIP_SUCCESS
                         : fail(NOVA_HIP_EINVAL, "line %d: %s takes %zu operands", op.line,
                                op.name.c_str(), n);
  };
  std::vector<Type> &R = op.result_types;
  // Operand ranks outside the op's form (include/nova_forms.h) are declined
  // before inference, with the table's reason.
  if (const nova_forms::RankForm *rf = nova_forms::rank_form(op.name.c_str())) {
    if ((int)T.size() == rf->nops)
      for (int i = 0; i < rf->nops; ++i) {
        const int r = (int)T[i].shape.size();
        if (r < rf->min_rank[i] || r > rf->max_rank[i])
          return fail(NOVA_HIP_EINVAL,
                      "line %d: %s: operand rank outside the form (see nova_forms.h) (not on "
                      "this path)",
                      op.line, op.name.c_str());
      }
  }
  if (!R.empty() && op.name != "nova.cast") return NOVA_HIP_SUCCESS;
  int32_t rc;
  if (op.name == "nova.matmul") {
    if ((rc = need(2))) return rc;
    const Type &a = T[0], &b = T[1];
    if (a.shape.size() < 2 || b.shape.size() < 2)
      return fail(NOVA_HIP_ESHAPE, "line %d: nova.matmul needs rank >= 2", op.line);
    Type r;
    r.shape = a.shape.size() >= b.shape.size() ? a.shape : b.shape;
    r.shape[r.shape.size() - 2] = a.shape[a.shape.size() - 2];
    r.shape[r.shape.size() - 1] = b.shape.back();
    // NovaOps.cpp:1198: bf16 x bf16 and f16 x f16 give f16; f32 gives f32.
    r.dt = a.dt == DT_F32 ? DT_F32 : DT_F16;
    R.push_back(r);
  } else if (op.name == "nova.linear") {
    if ((rc = need(3))) return rc;
    Type r = T[0];
    r.shape.back() = T[1].shape.back();
    R.push_back(r);
  } else if (op.name == "nova.gelu") {
    if ((rc = need(1))) return rc;
    R.push_back(T[0]);
  } else if (op.name == "nova.cast") {
    if ((rc = need(1))) return rc;
    if (R.size() != 1) return fail(NOVA_HIP_EINVAL, "line %d: nova.cast needs `-> type`", op.line);
  } else if (op.name == "nova.transpose") {
    if ((rc = need(1))) return rc;
    Type r = T[0];
    const int n = (int)r.shape.size();
    int a1 = op.attrs.count("axes1") ? atoi(op.attrs["axes1"].c_str()) : -1;
    int a2 = op.attrs.count("axes2") ? atoi(op.attrs["axes2"].c_str()) : -2;
    if (a1 < 0) a1 += n;
    if (a2 < 0) a2 += n;
    if (n < 2 || a1 < 0 || a2 < 0 || a1 >= n || a2 >= n)
      return fail(NOVA_HIP_ESHAPE, "line %d: bad transpose axes", op.line);
    std::swap(r.shape[a1], r.shape[a2]);
    op.attrs["axes1"] = std::to_string(a1);
    op.attrs["axes2"] = std::to_string(a2);
    R.push_back(r);
  } else if (op.name == "nova.layer_norm") {
    if ((rc = need(3))) return rc;
    Type s = T[0];
    s.shape.pop_back();
    R = {T[0], s, s};
  } else if (op.name == "nova.sce") {
    if ((rc = need(2))) return rc;
    Type loss;
    loss.shape = {1};
    loss.dt = T[0].dt;
    R = {T[0], loss};
  } else if (op.name == "nova.sce_backward") {
    if ((rc = need(2))) return rc;
    R = {T[0]};
  } else if (op.name == "nova.layer_norm_backward") {
    if ((rc = need(5))) return rc;
    R = {T[1], T[2], T[2]};
  } else if (op.name == "nova.linear_backward") {
    if ((rc = need(3))) return rc;
    Type gb = T[2];
    gb.shape = {T[2].shape.back()};
    R = {T[1], T[2], gb};
  } else if (op.name == "nova.matmul_backward") {
    if ((rc = need(3))) return rc;
    R = {T[1], T[2]};
  } else if (op.name == "nova.add" || op.name == "nova.sub" || op.name == "nova.mul" ||
             op.name == "nova.div") {
    // numpy-style broadcasting (Nova_BinaryOp, NovaOps.td:600-700)
    if ((rc = need(2))) return rc;
    const std::vector<int64_t> &a = T[0].shape, &b = T[1].shape;
    Type r;
    r.dt = T[0].dt;
    const size_t n = std::max(a.size(), b.size());
    r.shape.assign(n, 1);
    for (size_t i = 0; i < n; ++i) {
      const int64_t x = i < n - a.size() ? 1 : a[i - (n - a.size())];
      const int64_t y = i < n - b.size() ? 1 : b[i - (n - b.size())];
      if (x != y && x != 1 && y != 1)
        return fail(NOVA_HIP_ESHAPE, "line %d: %s shapes do not broadcast", op.line,
                    op.name.c_str());
      r.shape[i] = x == 1 ? y : x;
    }
    R.push_back(r);
  } else if (op.name == "nova.gelu_backward") {
    if ((rc = need(2))) return rc;
    R.push_back(T[1]);
  } else if (op.name == "nova.gather") {
    if ((rc = need(2))) return rc;
    Type r;
    r.dt = T[0].dt;
    r.shape = T[1].shape;
    for (size_t i = 1; i < T[0].shape.size(); ++i) r.shape.push_back(T[0].shape[i]);
    R.push_back(r);
  } else if (op.name == "nova.scatter_add") {
    if ((rc = need(3))) return rc;
    R.push_back(T[0]);
  } else if (op.name.compare(0, 11, "nova.reduce") == 0) {
    if ((rc = need(1))) return rc;
    std::vector<int> dims = reduce_dims(op, (int)T[0].shape.size());
    const bool keep = op.attrs.count("keepdims") && op.attrs.at("keepdims") == "true";
    Type r;
    r.dt = T[0].dt;
    for (int i = 0; i < (int)T[0].shape.size(); ++i) {
      bool red = false;
      for (int d : dims) red = red || d == i;
      if (!red) r.shape.push_back(T[0].shape[i]);
      else if (keep) r.shape.push_back(1);
    }
    R.push_back(r);
  } else if (op.name == "nova.reshape" || op.name == "nova.constant") {
    return fail(NOVA_HIP_EINVAL, "line %d: %s needs its result type", op.line, op.name.c_str());
  } else if (op.name.compare(0, 5, "nova.") == 0) {
    return fail(NOVA_HIP_EINVAL, "line %d: op '%s' is not part of this path's op surface",
                op.line, op.name.c_str());
  }
  return NOVA_HIP_SUCCESS;
}

// A single-result op written `%x = nova.sce` names the loss (result 1), as
// in the reference's own ltest/_sce.mlir.
void bind_results(Op &op) {
  if (op.name == "nova.sce" && op.results.size() == 1) op.results = {"", op.results[0]};
}

int32_t parse_func(const std::string &text, size_t at, size_t &end_out, Func &f) {
  const size_t name_at = text.find('@', at);
  const size_t lp = text.find('(', name_at);
  if (name_at == std::string::npos || lp == std::string::npos)
    return fail(NOVA_HIP_EINVAL, "line %d: malformed func.func", line_of(text, at));
  f.name = trim(text.substr(name_at + 1, lp - name_at - 1));
  const size_t rp = match_close(text, lp);
  if (rp == std::string::npos) return fail(NOVA_HIP_EINVAL, "unbalanced func signature");
  for (const std::string &a : split_top(text.substr(lp + 1, rp - lp - 1), ',')) {
    const size_t colon = a.find(':');
    if (colon == std::string::npos) return fail(NOVA_HIP_EINVAL, "bad argument '%s'", a.c_str());
    Type t;
    std::string ts = a.substr(colon + 1);
    const size_t brace = find_top(ts, '{');
    if (brace != std::string::npos) ts = ts.substr(0, brace);
    if (!parse_type(ts, t))
      return fail(NOVA_HIP_EINVAL, "line %d: unsupported argument type '%s'", line_of(text, lp),
                  trim(ts).c_str());
    f.arg_names.push_back(trim(a.substr(0, colon)));
    f.arg_types.push_back(t);
  }
  const size_t body_lb = text.find('{', rp);
  // `attributes {...}` before the body
  size_t lb = body_lb;
  const size_t attr = text.find("attributes", rp);
  if (attr != std::string::npos && attr < body_lb) lb = text.find('{', match_close(text, body_lb) + 1);
  const size_t rb = match_close(text, lb);
  if (lb == std::string::npos || rb == std::string::npos)
    return fail(NOVA_HIP_EINVAL, "line %d: func body not closed", line_of(text, at));
  end_out = rb + 1;
  // statements: lines joined while brackets are open
  const std::string body = text.substr(lb + 1, rb - lb - 1);
  size_t i = 0;
  std::string stmt;
  int depth = 0, stmt_line = 0;
  while (i <= body.size()) {
    const size_t nl = body.find('\n', i);
    const std::string ln = body.substr(i, nl == std::string::npos ? std::string::npos : nl - i);
    if (stmt.empty()) stmt_line = line_of(text, lb + 1 + i);
    for (char c : ln) depth += (c == '(' || c == '[' || c == '{') - (c == ')' || c == ']' || c == '}');
    stmt += " " + ln;
    // A statement also continues on a next line that starts with `outs`,
    // `->` or `:` (linalg ops written over several lines).
    bool cont = false;
    if (depth <= 0 && nl != std::string::npos) {
      size_t nx = nl + 1;
      while (nx < body.size() && (body[nx] == ' ' || body[nx] == '\t')) ++nx;
      cont = body.compare(nx, 4, "outs") == 0 || body.compare(nx, 2, "->") == 0 ||
             body.compare(nx, 1, ":") == 0;
    }
    if (depth <= 0 && !cont) {
      const std::string s = trim(stmt);
      stmt.clear();
      depth = 0;
      if (!s.empty()) {
        if (s.compare(0, 6, "return") == 0) {
          std::string r = trim(s.substr(6));
          const size_t colon = find_top(r, ':');
          f.rets = operand_names(colon == std::string::npos ? r : r.substr(0, colon));
        } else {
          Op op;
          int32_t rc = parse_op(s, stmt_line, op);
          if (rc) return rc;
          bind_results(op);
          if ((rc = infer(op))) return rc;
          f.ops.push_back(op);
        }
      }
    }
    if (nl == std::string::npos) break;
    i = nl + 1;
  }
  return NOVA_HIP_SUCCESS;
}

// ---- planning ----------------------------------------------------------------
struct View {
  int buf = -1;
  std::vector<int64_t> shape, strides;  // elements
  int dt = -1;                          // stored dtype
  int logical = -1;                     // dtype the program sees
  bool zero = false;                    // known all-zero (linalg.fill 0)
  int producer = -1;                    // step that writes the buffer, if a GEMM
};

struct Buffer {
  int64_t bytes = 0;
  int arg = -1;  // host argument index it is copied from, or -1
};

struct Step {
  // gemm, layer_norm, sce, sce_bwd, ln_bwd, lin_bwd, mm_bwd, zero, copy, view,
  // fill, binary, gelu, gelu_bwd, gather, scatter, reduce_sum, idx32
  std::string kind;
  std::vector<View> in, out;
  int epi = NOVA_HIP_EPI_NONE;  // GEMM epilogue; binary op code; index dtype
  int out_dt = DT_F32;
  std::string text;
  float value = 0.0f;           // fill value
  int64_t dims[3] = {0, 0, 0};  // reduce_sum: outer, reduced, inner
  bool acc_out = false;         // GEMM accumulating in its bf16 / f16 output dtype
  bool f32_mfma = false;        // f32 GEMM on the matrix cores (NOVA_HIP_GEMM_F32_MFMA)
  bool acc_c = false;           // GEMM summing from its output's data (NOVA_HIP_GEMM_ACC_C)
};

int64_t numel_of(const std::vector<int64_t> &shape) {
  int64_t n = 1;
  for (int64_t d : shape) n *= d;
  return n;
}

std::vector<int64_t> dense_strides(const std::vector<int64_t> &shape) {
  std::vector<int64_t> st(shape.size(), 1);
  for (int i = (int)shape.size() - 2; i >= 0; --i) st[i] = st[i + 1] * shape[i + 1];
  return st;
}

bool is_dense(const View &v) { return v.strides == dense_strides(v.shape); }

// Dims [0, n - R) of v fold into dim n - R of a rank-R descriptor: each
// folded dim's stride is the next one's stride times its size (dims of size
// one are free).
bool leading_dims_fold(const View &v, int R) {
  const int n = (int)v.shape.size();
  for (int j = n - R - 1; j >= 0; --j)
    if (v.shape[j] > 1 && v.strides[j] != v.strides[j + 1] * v.shape[j + 1]) return false;
  return true;
}

struct Plan {
  std::vector<Buffer> bufs;
  std::vector<Step> steps;
  std::vector<View> results;
  std::vector<int> out_args;  // writable memref arguments: arg index per materialize step
};

std::string view_str(const View &v) {
  std::string s = "b" + std::to_string(v.buf) + "[";
  for (size_t i = 0; i < v.shape.size(); ++i) s += (i ? "," : "") + std::to_string(v.shape[i]);
  s += "]";
  s += dt_name(v.dt);
  if (!is_dense(v)) {
    s += " strides(";
    for (size_t i = 0; i < v.strides.size(); ++i)
      s += (i ? "," : "") + std::to_string(v.strides[i]);
    s += ")";
  }
  return s;
}

struct Planner {
  const Func &f;
  Plan plan;
  std::map<std::string, View> env;
  std::map<std::string, int> uses;
  std::map<std::string, std::string> consts;
  std::set<int> empty_bufs;  // buffers of tensor.empty results
  std::set<std::string> empty_vals;  // tensor.empty results (uninitialised data)
  std::set<std::string> ones;  // splat 1.0 constants whose every use is an identity multiply
  bool f32_mfma = false;       // plan f32 GEMMs onto the matrix cores

  explicit Planner(const Func &fn, bool mfma = false) : f(fn), f32_mfma(mfma) {}

  int new_buf(const Type &t, int arg = -1) {
    Buffer b;
    b.bytes = t.numel() * dt_size(t.dt);
    b.arg = arg;
    plan.bufs.push_back(b);
    return (int)plan.bufs.size() - 1;
  }
  View fresh(const Type &t) {
    View v;
    v.buf = new_buf(t);
    v.shape = t.shape;
    v.strides = dense_strides(t.shape);
    v.dt = v.logical = t.dt;
    return v;
  }
  int32_t get(const Op &op, size_t i, View &v) {
    auto it = env.find(op.operands[i]);
    if (it == env.end())
      return fail(NOVA_HIP_EINVAL, "line %d: %s uses undefined value %s", op.line, op.name.c_str(),
                  op.operands[i].c_str());
    v = it->second;
    return NOVA_HIP_SUCCESS;
  }
  int32_t need_f32(const Op &op, const View &v, const char *what) {
    if (v.dt != DT_F32)
      return fail(NOVA_HIP_EDTYPE,
                  "line %d: %s of %s must be stored f32 (a cast from %s is folded only into GEMM "
                  "operands)",
                  op.line, what, op.name.c_str(), dt_name(v.dt));
    return NOVA_HIP_SUCCESS;
  }
  // The op's form against the table both carriers of the rewrite consult
  // (include/nova_forms.h): each operand's stored and logical element type
  // and shape, the result element types, and the attributes the form
  // depends on.
  int32_t form(const Op &op, std::initializer_list<const View *> vs,
               const nova_forms::Attrs &at = nova_forms::Attrs(), const char *name = nullptr) {
    nova_forms::Operand o[nova_forms::kMaxOperands];
    int n = 0;
    for (const View *v : vs) {
      if (n == nova_forms::kMaxOperands) break;
      o[n].stored = v->dt;
      o[n].logical = v->logical;
      o[n].rank = (int)v->shape.size();
      o[n].shape = v->shape.data();
      ++n;
    }
    int rd[8];
    int nr = 0;
    for (const Type &t : op.result_types)
      if (nr < 8) rd[nr++] = t.dt;
    const char *why = nova_forms::check(name ? name : op.name.c_str(), n, o, nr, rd, at);
    if (why)
      return fail(NOVA_HIP_EINVAL, "line %d: %s: %s (not on this path)", op.line, op.name.c_str(),
                  why);
    return NOVA_HIP_SUCCESS;
  }
  int32_t need_dense_f32(const Op &op, const View &v, const char *what) {
    int32_t rc = need_f32(op, v, what);
    if (rc) return rc;
    if (!is_dense(v))
      return fail(NOVA_HIP_ESTRIDE, "line %d: %s of %s is a transposed view (not on this path)",
                  op.line, what, op.name.c_str());
    return NOVA_HIP_SUCCESS;
  }
  // Labels / indices as i32: non-i32 index types get a widening step (the
  // reference zero-extends narrow label types, NovaToLinalgGeneric.cpp:801-1010).
  int32_t as_i32(const Op &op, View &t) {
    if (t.dt == DT_I32) return NOVA_HIP_SUCCESS;
    if (!is_index_dt(t.dt) || !is_dense(t))
      return fail(NOVA_HIP_EDTYPE, "line %d: %s targets must be an integer tensor", op.line,
                  op.name.c_str());
    Step s;
    s.kind = "idx32";
    s.in = {t};
    s.out = {fresh(Type{t.shape, DT_I32, false})};
    s.text = std::string(dt_name(t.dt)) + " labels -> _mlir_ciface_nova_hip_index_to_i32(" +
             view_str(t) + ") -> " + view_str(s.out[0]);
    plan.steps.push_back(s);
    t = s.out[0];
    return NOVA_HIP_SUCCESS;
  }
  // The single consumer of `name` if it has exactly one use, else null.
  const Op *sole_user(const std::string &name, size_t from) {
    if (uses[name] != 1) return nullptr;
    for (size_t k = from; k < f.ops.size(); ++k)
      for (const std::string &o : f.ops[k].operands)
        if (o == name) return &f.ops[k];
    return nullptr;
  }

  // Every use of `name` (from op index `from` on) is a nova.mul whose other
  // operand is an f32 value of the result's shape (so the multiply by a
  // broadcast splat leaves it unchanged), and it is not returned.
  bool identity_muls_only(const std::string &name, size_t from) {
    if (uses[name] == 0) return false;
    for (const std::string &r : f.rets)
      if (r == name) return false;
    int seen = 0;
    for (size_t k = from; k < f.ops.size(); ++k) {
      const Op &o = f.ops[k];
      for (size_t i = 0; i < o.operands.size(); ++i) {
        if (o.operands[i] != name) continue;
        if (o.name != "nova.mul" || o.operands.size() != 2 || o.operands[0] == o.operands[1])
          return false;
        const size_t other = 1 - i;
        if (other >= o.operand_types.size() || o.result_types.empty()) return false;
        const Type &ot = o.operand_types[other];
        if (ot.dt != DT_F32 || ot.shape != o.result_types[0].shape) return false;
        ++seen;
      }
    }
    return seen == uses[name];
  }

  // A GEMM-family step writing `out` (reusing its buffer when it has one of
  // the output dtype, as a linalg init does); then folds of a following
  // gelu / narrowing cast.
  int32_t emit_gemm(const Op &op, size_t idx, View a, View b, const View *bias, View out,
                    std::set<const Op *> &folded) {
    if (a.dt != b.dt)
      return fail(NOVA_HIP_EDTYPE, "line %d: %s operands are stored as %s and %s", op.line,
                  op.name.c_str(), dt_name(a.dt), dt_name(b.dt));
    if (a.dt > DT_F16)
      return fail(NOVA_HIP_EDTYPE, "line %d: %s on %s is not on this path", op.line,
                  op.name.c_str(), dt_name(a.dt));
    if (a.dt == DT_F32 && out.dt != DT_F32)
      return fail(NOVA_HIP_EDTYPE, "line %d: f32 operands give f32 results only", op.line);
    // A bf16 / f16 result is a linalg.matmul with narrow outs, whose body
    // runs in the outs type (NovaToLinalg.cpp:1027-1049): the accumulator is
    // that dtype.  Only the same-dtype form is on this path: a bf16 x bf16
    // nova.matmul infers f16 (NovaOps.cpp:1198), and what linalg's element
    // cast does between two 16-bit float types is not pinned here.
    const bool narrow = out.dt != DT_F32;
    if (narrow) {
      if (a.logical != a.dt || b.logical != b.dt || a.dt != out.dt)
        return fail(NOVA_HIP_EDTYPE,
                    "line %d: %s of %s operands with a %s result accumulates in %s through a "
                    "%s -> %s element cast that is not on this path (spell the f32-accumulate "
                    "form: nova.cast the operands to f32, or f32 linalg outs)",
                    op.line, op.name.c_str(), dt_name(a.logical), dt_name(out.dt),
                    dt_name(out.dt), dt_name(a.logical), dt_name(out.dt));
      if (bias && (bias->dt != out.dt || bias->logical != bias->dt))
        return fail(NOVA_HIP_EDTYPE, "line %d: %s with a %s accumulator needs a %s bias",
                    op.line, op.name.c_str(), dt_name(out.dt), dt_name(out.dt));
    }
    Step s;
    s.kind = "gemm";
    s.in = {a, b};
    if (bias) s.in.push_back(*bias);
    s.epi = bias ? NOVA_HIP_EPI_BIAS : NOVA_HIP_EPI_NONE;
    s.out_dt = out.dt;
    s.acc_out = narrow;
    s.f32_mfma = f32_mfma && a.dt == DT_F32;
    std::string name = op.results[0];
    std::string fused = op.name;
    // (GELU and casts fold only into an f32 accumulator.)
    const Op *u = narrow ? nullptr : sole_user(name, idx + 1);
    if (u && u->name == "nova.gelu") {
      s.epi = bias ? NOVA_HIP_EPI_BIAS_GELU : NOVA_HIP_EPI_GELU;
      folded.insert(u);
      fused += " + nova.gelu";
      env[u->results[0]] = out;  // placeholder, fixed below
      name = u->results[0];
      u = sole_user(name, idx + 1);
    }
    if (u && u->name == "nova.cast" && u->result_types[0].dt != DT_F32 && out.dt == DT_F32 &&
        u->result_types[0].dt <= DT_F16) {
      s.out_dt = u->result_types[0].dt;
      folded.insert(u);
      fused += " + nova.cast";
      name = u->results[0];
    }
    if (out.buf < 0 || out.dt != s.out_dt) out = fresh(Type{out.shape, s.out_dt, false});
    out.zero = false;
    out.producer = (int)plan.steps.size();
    s.out = {out};
    char buf[512];
    snprintf(buf, sizeof(buf), "%s -> _mlir_ciface_nova_hip_gemm(%s, %s%s%s) -> %s epilogue=%s",
             fused.c_str(), view_str(a).c_str(), view_str(b).c_str(), bias ? ", bias " : "",
             bias ? view_str(*bias).c_str() : "", view_str(out).c_str(),
             s.epi == NOVA_HIP_EPI_NONE ? "none" : s.epi == NOVA_HIP_EPI_BIAS ? "bias"
             : s.epi == NOVA_HIP_EPI_BIAS_GELU ? "bias+gelu" : "gelu");
    s.text = buf;
    if (narrow) s.text += std::string(" accumulate=") + dt_name(out.dt);
    if (s.f32_mfma) s.text += " f32=mfma";
    plan.steps.push_back(s);
    env[op.results[0]] = out;
    env[name] = out;
    return NOVA_HIP_SUCCESS;
  }

  // linalg.matmul / batch_matmul whose outs holds data: the result is
  // outs + A . B, each sum starting from outs' element (NOVA_HIP_GEMM_ACC_C,
  // the exact kernel).  The sums go into outs' own buffer when this op is
  // the only reader of a dense intermediate; otherwise into a copy of it,
  // so that a function argument or a value read again keeps its data.
  int32_t emit_gemm_acc(const Op &op, const View &a, const View &b, View c) {
    if (empty_vals.count(op.operands[2]))
      return fail(NOVA_HIP_EINVAL, "line %d: %s reads an uninitialised tensor.empty as its outs",
                  op.line, op.name.c_str());
    if (!is_dense(c))
      return fail(NOVA_HIP_ESTRIDE, "line %d: %s outs is a strided view (not on this path)",
                  op.line, op.name.c_str());
    const bool narrow = c.dt != DT_F32;
    // Another value naming the same buffer (a reshape view, a value the
    // buffer was handed on from) may still be read: then copy too.
    bool shared = plan.bufs[c.buf].arg >= 0 || uses[op.operands[2]] != 1;
    for (const auto &kv : env) shared = shared || (kv.first != op.operands[2] && kv.second.buf == c.buf);
    View out = c;
    if (shared) {
      out = fresh(Type{c.shape, c.dt, false});
      Step cp;
      cp.kind = "copy";
      cp.in = {c};
      cp.out = {out};
      cp.text = op.name + " outs -> hipMemcpyAsync(" + view_str(out) + " <- " + view_str(c) + ")";
      plan.steps.push_back(cp);
    }
    out.zero = false;
    out.producer = (int)plan.steps.size();
    Step s;
    s.kind = "gemm";
    s.in = {a, b};
    s.out = {out};
    s.out_dt = out.dt;
    s.acc_out = narrow;
    s.acc_c = true;
    s.text = op.name + " -> _mlir_ciface_nova_hip_gemm(" + view_str(a) + ", " + view_str(b) +
             ") -> " + view_str(out) + " accumulate-into=" + dt_name(out.dt);
    plan.steps.push_back(s);
    env[op.results[0]] = out;
    return NOVA_HIP_SUCCESS;
  }

  int32_t run() {
    for (size_t i = 0; i < f.arg_names.size(); ++i) {
      View v;
      v.buf = new_buf(f.arg_types[i], (int)i);
      v.shape = f.arg_types[i].shape;
      v.strides = dense_strides(v.shape);
      v.dt = v.logical = f.arg_types[i].dt;
      env[f.arg_names[i]] = v;
    }
    for (const Op &op : f.ops)
      for (const std::string &o : op.operands) uses[o]++;
    for (const std::string &r : f.rets) uses[r]++;
    std::set<const Op *> folded;
    int32_t rc;
    for (size_t k = 0; k < f.ops.size(); ++k) {
      const Op &op = f.ops[k];
      if (folded.count(&op)) continue;
      const std::string &n = op.name;
      if (n == "arith.constant") {
        consts[op.results[0]] = op.literal;
      } else if (n == "tensor.empty") {
        env[op.results[0]] = fresh(op.result_types[0]);
        empty_bufs.insert(env[op.results[0]].buf);
        empty_vals.insert(op.results[0]);
      } else if (n == "bufferization.to_tensor") {
        View v;
        if ((rc = get(op, 0, v))) return rc;
        env[op.results[0]] = v;
      } else if (n == "linalg.fill") {
        View dst;
        if ((rc = get(op, 1, dst))) return rc;
        const std::string c = consts.count(op.operands[0]) ? consts[op.operands[0]] : "";
        if (c.empty() || strtod(c.c_str(), nullptr) != 0.0)
          return fail(NOVA_HIP_EINVAL, "line %d: linalg.fill with a value other than 0 is not on this path",
                      op.line);
        // The fill's result is a new tensor.  It takes over its destination's
        // buffer only when that is a tensor.empty used by nothing else;
        // otherwise (a function argument, a value read again later) it gets
        // a buffer of its own, so the fill and the GEMMs writing into it
        // leave the destination as it was.
        if (!empty_bufs.count(dst.buf) || uses[op.operands[1]] != 1) {
          const int dt = dst.logical;
          dst = fresh(Type{dst.shape, dt, false});
        }
        dst.zero = true;
        env[op.results[0]] = dst;
        // The fill only matters if its result is read by something other
        // than a matmul's outs (which the GEMM overwrites).
        bool only_outs = true;
        for (size_t j = k + 1; j < f.ops.size(); ++j)
          for (size_t o = 0; o < f.ops[j].operands.size(); ++o)
            if (f.ops[j].operands[o] == op.results[0] &&
                !((f.ops[j].name == "linalg.matmul" || f.ops[j].name == "linalg.batch_matmul") &&
                  o == 2))
              only_outs = false;
        for (const std::string &r : f.rets) only_outs = only_outs && r != op.results[0];
        if (!only_outs) {
          Step s;
          s.kind = "zero";
          s.out = {dst};
          s.text = numel_of(dst.shape) * dt_size(dst.dt) % 4 == 0
                       ? "linalg.fill 0 -> _mlir_ciface_nova_hip_fill_f32(" + view_str(dst) + ", 0)"
                       : "linalg.fill 0 -> hipMemsetAsync(" + view_str(dst) + ")";
          plan.steps.push_back(s);
        }
      } else if (n == "linalg.matmul" || n == "linalg.batch_matmul") {
        View a, b, c;
        if ((rc = get(op, 0, a)) || (rc = get(op, 1, b)) || (rc = get(op, 2, c))) return rc;
        nova_forms::Attrs at;
        at.outs_zero = c.zero;
        if ((rc = form(op, {&a, &b, &c}, at))) return rc;
        if (!c.zero) {
          if ((rc = emit_gemm_acc(op, a, b, c))) return rc;
          continue;
        }
        if (op.result_types[0].dt != DT_F32 && a.dt != op.result_types[0].dt)
          return fail(NOVA_HIP_EDTYPE, "line %d: %s with %s outs is not on this path", op.line,
                      n.c_str(), dt_name(op.result_types[0].dt));
        // The product writes its outs buffer in place only when this GEMM is
        // the fill result's sole user; two GEMMs over one (CSE'd) fill each
        // get a buffer of their own.
        if (uses[op.operands[2]] != 1) c.buf = -1;
        if ((rc = emit_gemm(op, k, a, b, nullptr, c, folded))) return rc;
      } else if (n == "nova.matmul") {
        View a, b;
        if ((rc = get(op, 0, a)) || (rc = get(op, 1, b)) || (rc = form(op, {&a, &b}))) return rc;
        View out;
        out.shape = op.result_types[0].shape;
        out.dt = op.result_types[0].dt;
        if ((rc = emit_gemm(op, k, a, b, nullptr, out, folded))) return rc;
      } else if (n == "nova.linear") {
        View x, w, bias;
        if ((rc = get(op, 0, x)) || (rc = get(op, 1, w)) || (rc = get(op, 2, bias)) ||
            (rc = form(op, {&x, &w, &bias})))
          return rc;
        View out;
        out.shape = op.result_types[0].shape;
        out.dt = op.result_types[0].dt;
        if ((rc = emit_gemm(op, k, x, w, &bias, out, folded))) return rc;
      } else if (n == "nova.gelu") {
        // not folded: its input has other uses (e.g. a gelu_backward)
        View x;
        if ((rc = get(op, 0, x)) || (rc = form(op, {&x})) || (rc = need_dense_f32(op, x, "input")))
          return rc;
        Step s;
        s.kind = "gelu";
        s.in = {x};
        s.out = {fresh(op.result_types[0])};
        s.text = "nova.gelu -> _mlir_ciface_nova_hip_gelu_f32(" + view_str(x) + ") -> " +
                 view_str(s.out[0]);
        env[op.results[0]] = s.out[0];
        plan.steps.push_back(s);
      } else if (n == "nova.gelu_backward") {
        View go, x;
        if ((rc = get(op, 0, go)) || (rc = get(op, 1, x)) || (rc = form(op, {&go, &x})) ||
            (rc = need_dense_f32(op, go, "grad_out")) || (rc = need_dense_f32(op, x, "input")))
          return rc;
        if (numel_of(go.shape) != numel_of(x.shape))
          return fail(NOVA_HIP_ESHAPE, "line %d: nova.gelu_backward operand sizes differ", op.line);
        Step s;
        s.kind = "gelu_bwd";
        s.in = {go, x};
        s.out = {fresh(op.result_types[0])};
        s.text = "nova.gelu_backward -> _mlir_ciface_nova_hip_gelu_backward_f32(" + view_str(go) +
                 ", " + view_str(x) + ") -> " + view_str(s.out[0]);
        env[op.results[0]] = s.out[0];
        plan.steps.push_back(s);
      } else if (n == "nova.mul" && (ones.count(op.operands[0]) || ones.count(op.operands[1]))) {
        const size_t keep = ones.count(op.operands[0]) ? 1 : 0;
        View v, one;
        if ((rc = get(op, keep, v)) || (rc = get(op, 1 - keep, one)) ||
            (rc = form(op, {keep ? &one : &v, keep ? &v : &one})))
          return rc;
        v.producer = -1;
        env[op.results[0]] = v;
        plan.steps.push_back(Step{"view", {}, {}, 0, 0,
                                  "nova.mul by splat 1.0 -> view " + view_str(v)});
      } else if (n == "nova.add" || n == "nova.sub" || n == "nova.mul" || n == "nova.div") {
        View a, b;
        if ((rc = get(op, 0, a)) || (rc = get(op, 1, b)) || (rc = form(op, {&a, &b})) ||
            (rc = need_dense_f32(op, a, "lhs")) || (rc = need_dense_f32(op, b, "rhs")))
          return rc;
        if (op.result_types[0].shape.size() > 4)
          return fail(NOVA_HIP_ESHAPE, "line %d: %s above rank 4", op.line, n.c_str());
        Step s;
        s.kind = "binary";
        s.epi = n == "nova.add" ? NOVA_HIP_BIN_ADD : n == "nova.sub" ? NOVA_HIP_BIN_SUB
              : n == "nova.mul" ? NOVA_HIP_BIN_MUL : NOVA_HIP_BIN_DIV;
        s.in = {a, b};
        s.out = {fresh(op.result_types[0])};
        s.text = n + " -> _mlir_ciface_nova_hip_binary_f32(" + view_str(a) + ", " + view_str(b) +
                 ") -> " + view_str(s.out[0]);
        env[op.results[0]] = s.out[0];
        plan.steps.push_back(s);
      } else if (n == "nova.constant") {
        const std::string v = op.attrs.count("value") ? op.attrs.at("value") : "";
        const Type &t = op.result_types[0];
        if (v.compare(0, 6, "dense<") != 0 || v.find('[') != std::string::npos)
          return fail(NOVA_HIP_EINVAL,
                      "line %d: nova.constant other than a splat dense<value> is not on this path",
                      op.line);
        if (t.dt != DT_F32)
          return fail(NOVA_HIP_EDTYPE, "line %d: nova.constant of %s is not on this path", op.line,
                      dt_name(t.dt));
        if ((rc = form(op, {}))) return rc;
        const float value = strtof(v.c_str() + 6, nullptr);
        // x * 1.0 == x for every f32 x: a splat 1.0 whose every use is a
        // nova.mul that leaves the other operand's shape unchanged needs
        // neither the fill nor the multiplies (each becomes a view).
        if (value == 1.0f && identity_muls_only(op.results[0], k + 1)) {
          ones.insert(op.results[0]);
          View one;
          one.shape = t.shape;
          one.strides = dense_strides(t.shape);
          one.dt = one.logical = DT_F32;
          env[op.results[0]] = one;  // never read: no buffer
          plan.steps.push_back(Step{"view", {}, {}, 0, 0,
                                    "nova.constant splat 1 -> elided (identity multiplies only)"});
          continue;
        }
        Step s;
        s.kind = "fill";
        s.out = {fresh(t)};
        s.value = value;
        char buf[64];
        snprintf(buf, sizeof(buf), "%g", (double)s.value);
        s.text = std::string("nova.constant splat ") + buf + " -> _mlir_ciface_nova_hip_fill_f32(" +
                 view_str(s.out[0]) + ")";
        env[op.results[0]] = s.out[0];
        plan.steps.push_back(s);
      } else if (n == "nova.reshape") {
        View v;
        if ((rc = get(op, 0, v))) return rc;
        const Type &t = op.result_types[0];
        if (!is_dense(v) || v.dt != v.logical)
          return fail(NOVA_HIP_ESTRIDE,
                      "line %d: nova.reshape of a view (transpose / folded cast) is not on this path",
                      op.line);
        if (numel_of(t.shape) != numel_of(v.shape))
          return fail(NOVA_HIP_ESHAPE, "line %d: nova.reshape changes the element count", op.line);
        v.shape = t.shape;
        v.strides = dense_strides(t.shape);
        v.producer = -1;
        env[op.results[0]] = v;
        plan.steps.push_back(Step{"view", {}, {}, 0, 0, "nova.reshape -> view " + view_str(v)});
      } else if (n == "nova.gather") {
        View t, idx;
        nova_forms::Attrs at;
        at.axis = op.attrs.count("axis") ? atoi(op.attrs.at("axis").c_str()) : 0;
        if (at.axis < 0) at.axis += (int)op.operand_types[0].shape.size();
        if ((rc = get(op, 0, t)) || (rc = get(op, 1, idx)) || (rc = form(op, {&t, &idx}, at)) ||
            (rc = need_dense_f32(op, t, "input")))
          return rc;
        if ((op.attrs.count("axis") && atoi(op.attrs.at("axis").c_str()) != 0) || t.shape.size() != 2)
          return fail(NOVA_HIP_EINVAL, "line %d: nova.gather of a 2-D table along axis 0 only",
                      op.line);
        if (!is_index_dt(idx.dt) || !is_dense(idx))
          return fail(NOVA_HIP_EDTYPE, "line %d: nova.gather indices must be i16 / i32 / i64",
                      op.line);
        Step s;
        s.kind = "gather";
        s.epi = idx.dt;
        s.in = {t, idx};
        s.out = {fresh(op.result_types[0])};
        s.text = "nova.gather -> _mlir_ciface_nova_hip_gather_f32(" + view_str(t) + ", " +
                 view_str(idx) + ") -> " + view_str(s.out[0]);
        env[op.results[0]] = s.out[0];
        plan.steps.push_back(s);
      } else if (n == "nova.scatter_add") {
        View base, idx, src;
        nova_forms::Attrs at;
        at.axis = op.attrs.count("axis") ? atoi(op.attrs.at("axis").c_str()) : 0;
        if (at.axis < 0) at.axis += (int)op.operand_types[0].shape.size();
        if ((rc = get(op, 0, base)) || (rc = get(op, 1, idx)) || (rc = get(op, 2, src)) ||
            (rc = form(op, {&base, &idx, &src}, at)) || (rc = need_dense_f32(op, base, "input")) ||
            (rc = need_dense_f32(op, src, "src")))
          return rc;
        if ((op.attrs.count("axis") && atoi(op.attrs.at("axis").c_str()) != 0) ||
            base.shape.size() != 2)
          return fail(NOVA_HIP_EINVAL, "line %d: nova.scatter_add into a 2-D input along axis 0 only",
                      op.line);
        if (!is_index_dt(idx.dt) || !is_dense(idx))
          return fail(NOVA_HIP_EDTYPE, "line %d: nova.scatter_add indices must be i16 / i32 / i64",
                      op.line);
        if (numel_of(src.shape) != numel_of(idx.shape) * base.shape[1])
          return fail(NOVA_HIP_ESHAPE, "line %d: nova.scatter_add src is not [indices, %lld]",
                      op.line, (long long)base.shape[1]);
        // the op's result is a new tensor: the input copied, then the adds
        View out = fresh(op.result_types[0]);
        Step c;
        c.kind = "copy";
        c.in = {base};
        c.out = {out};
        c.text = "nova.scatter_add input -> hipMemcpyAsync(" + view_str(out) + " <- " +
                 view_str(base) + ")";
        plan.steps.push_back(c);
        Step s;
        s.kind = "scatter";
        s.epi = idx.dt;
        s.in = {idx, src};
        s.out = {out};
        s.text = "nova.scatter_add -> _mlir_ciface_nova_hip_scatter_add_f32(" + view_str(out) +
                 ", " + view_str(idx) + ", " + view_str(src) + ")";
        env[op.results[0]] = out;
        plan.steps.push_back(s);
      } else if (n.compare(0, 11, "nova.reduce") == 0) {
        View x;
        if ((rc = get(op, 0, x)) || (rc = need_dense_f32(op, x, "input"))) return rc;
        if (n != "nova.reduce<sum>")
          return fail(NOVA_HIP_EINVAL, "line %d: %s: only the sum reduction is on this path",
                      op.line, n.c_str());
        if (op.attrs.count("ignore_nan") && op.attrs.at("ignore_nan") == "true")
          return fail(NOVA_HIP_EINVAL, "line %d: nova.reduce ignore_nan is not on this path",
                      op.line);
        std::vector<int> dims = reduce_dims(op, (int)x.shape.size());
        std::sort(dims.begin(), dims.end());
        nova_forms::Attrs at;
        for (size_t i = 1; i < dims.size(); ++i) at.adjacent = at.adjacent && dims[i] == dims[i - 1] + 1;
        if ((rc = form(op, {&x}, at))) return rc;
        if (dims.empty() || dims[0] < 0 || dims.back() >= (int)x.shape.size())
          return fail(NOVA_HIP_EINVAL, "line %d: bad nova.reduce dimension", op.line);
        Step s;
        s.kind = "reduce_sum";
        s.dims[0] = numel_of(std::vector<int64_t>(x.shape.begin(), x.shape.begin() + dims[0]));
        s.dims[1] = numel_of(std::vector<int64_t>(x.shape.begin() + dims[0],
                                                  x.shape.begin() + dims.back() + 1));
        s.dims[2] = numel_of(std::vector<int64_t>(x.shape.begin() + dims.back() + 1, x.shape.end()));
        s.in = {x};
        s.out = {fresh(op.result_types[0])};
        s.text = "nova.reduce<sum> -> _mlir_ciface_nova_hip_reduce_sum_f32(" + view_str(x) +
                 " as [" + std::to_string(s.dims[0]) + "," + std::to_string(s.dims[1]) + "," +
                 std::to_string(s.dims[2]) + "]) -> " + view_str(s.out[0]);
        env[op.results[0]] = s.out[0];
        plan.steps.push_back(s);
      } else if (n == "nova.transpose") {
        View v;
        if ((rc = get(op, 0, v))) return rc;
        const int a1 = atoi(op.attrs.at("axes1").c_str()), a2 = atoi(op.attrs.at("axes2").c_str());
        std::swap(v.shape[a1], v.shape[a2]);
        std::swap(v.strides[a1], v.strides[a2]);
        v.producer = -1;
        env[op.results[0]] = v;
        plan.steps.push_back(Step{"view", {}, {}, 0, 0,
                                  "nova.transpose -> view " + view_str(v)});
      } else if (n == "nova.cast") {
        View v;
        if ((rc = get(op, 0, v))) return rc;
        const int to = op.result_types[0].dt;
        if (to == v.logical) {
          env[op.results[0]] = v;
        } else if (to == DT_F32 && (v.logical == DT_BF16 || v.logical == DT_F16)) {
          v.logical = DT_F32;  // exact widening: consumers read the stored narrow data
          env[op.results[0]] = v;
          plan.steps.push_back(Step{"view", {}, {}, 0, 0,
                                    std::string("nova.cast ") + dt_name(v.dt) +
                                        " -> f32 folded: consumers read " + view_str(v)});
        } else {
          return fail(NOVA_HIP_EINVAL,
                      "line %d: nova.cast %s -> %s is not foldable here (narrowing casts fold "
                      "only into the GEMM whose sole use they are)",
                      op.line, dt_name(v.logical), dt_name(to));
        }
      } else if (n == "nova.layer_norm") {
        View x, g, b;
        if ((rc = get(op, 0, x)) || (rc = get(op, 1, g)) || (rc = get(op, 2, b)) ||
            (rc = form(op, {&x, &g, &b})))
          return rc;
        if ((rc = need_f32(op, x, "input")) || (rc = need_f32(op, g, "gamma")) ||
            (rc = need_f32(op, b, "beta")))
          return rc;
        Step s;
        s.kind = "layer_norm";
        s.in = {x, g, b};
        s.out = {fresh(op.result_types[0]), fresh(op.result_types[1]), fresh(op.result_types[2])};
        s.text = "nova.layer_norm -> _mlir_ciface_nova_hip_layer_norm_f32(" + view_str(x) +
                 ") -> " + view_str(s.out[0]) + ", " + view_str(s.out[1]) + ", " +
                 view_str(s.out[2]);
        for (int r = 0; r < 3 && r < (int)op.results.size(); ++r) env[op.results[r]] = s.out[r];
        plan.steps.push_back(s);
      } else if (n == "nova.sce") {
        View x, t;
        if ((rc = get(op, 0, x)) || (rc = get(op, 1, t)) || (rc = form(op, {&x, &t}))) return rc;
        if ((rc = need_f32(op, x, "logits")) || (rc = as_i32(op, t))) return rc;
        // nova.sce whose softmax feeds only a nova.sce_backward over the same
        // labels: one fused launch writes the loss and the gradient, and the
        // softmax is never materialised.
        const Op *bw = op.results[0].empty() ? nullptr : sole_user(op.results[0], k + 1);
        if (bw && bw->name == "nova.sce_backward" && bw->operands.size() == 2 &&
            bw->operands[0] == op.results[0] && bw->operands[1] == op.operands[1] &&
            (!bw->attrs.count("dim") || atoi(bw->attrs.at("dim").c_str()) == -1 ||
             atoi(bw->attrs.at("dim").c_str()) == (int)x.shape.size() - 1)) {
          Step s;
          s.kind = "sce_fwd_bwd";
          s.in = {x, t};
          s.out = {fresh(bw->result_types[0]), fresh(op.result_types[1])};
          s.text = "nova.sce + nova.sce_backward -> _mlir_ciface_nova_hip_sce_fwd_bwd_f32(" +
                   view_str(x) + ", " + view_str(t) + ") -> " + view_str(s.out[0]) + ", " +
                   view_str(s.out[1]) + " (softmax not materialised)";
          folded.insert(bw);
          env[bw->results[0]] = s.out[0];
          env[op.results[1]] = s.out[1];
          plan.steps.push_back(s);
          continue;
        }
        Step s;
        s.kind = "sce";
        s.in = {x, t};
        const bool want_sm = !op.results[0].empty() && uses[op.results[0]] > 0;
        View sm;
        if (want_sm) sm = fresh(op.result_types[0]);
        s.out = {sm, fresh(op.result_types[1])};
        s.text = "nova.sce -> _mlir_ciface_nova_hip_sce_f32(" + view_str(x) + ", " + view_str(t) +
                 ") -> " + (want_sm ? view_str(sm) : std::string("(softmax unused)")) + ", " +
                 view_str(s.out[1]);
        if (want_sm) env[op.results[0]] = sm;
        env[op.results[1]] = s.out[1];
        plan.steps.push_back(s);
      } else if (n == "nova.sce_backward") {
        View sm, t;
        nova_forms::Attrs at;
        if (op.attrs.count("dim")) {
          at.dim = atoi(op.attrs.at("dim").c_str());
          if (at.dim < 0) at.dim += (int)op.operand_types[0].shape.size();
          if (at.dim == (int)op.operand_types[0].shape.size() - 1) at.dim = -1;
        }
        if ((rc = get(op, 0, sm)) || (rc = get(op, 1, t)) || (rc = form(op, {&sm, &t}, at)))
          return rc;
        if ((rc = need_f32(op, sm, "softmax")) || (rc = as_i32(op, t))) return rc;
        if (op.attrs.count("dim")) {
          const int d = atoi(op.attrs.at("dim").c_str());
          if (d != -1 && d != (int)sm.shape.size() - 1)
            return fail(NOVA_HIP_EINVAL, "line %d: nova.sce_backward over dim %d (class dim last only)",
                        op.line, d);
        }
        Step s;
        s.kind = "sce_bwd";
        s.in = {sm, t};
        s.out = {fresh(op.result_types[0])};
        s.text = "nova.sce_backward -> _mlir_ciface_nova_hip_sce_backward_f32(" + view_str(sm) +
                 ") -> " + view_str(s.out[0]);
        env[op.results[0]] = s.out[0];
        plan.steps.push_back(s);
      } else if (n == "nova.layer_norm_backward") {
        View gy, x, g, S, r;
        if ((rc = get(op, 0, gy)) || (rc = get(op, 1, x)) || (rc = get(op, 2, g)) ||
            (rc = get(op, 3, S)) || (rc = get(op, 4, r)) || (rc = form(op, {&gy, &x, &g, &S, &r})))
          return rc;
        for (const View *v : {&gy, &x, &g, &S, &r})
          if ((rc = need_f32(op, *v, "operand"))) return rc;
        Step s;
        s.kind = "ln_bwd";
        s.in = {gy, x, g, S, r};
        s.out = {fresh(op.result_types[0]), fresh(op.result_types[1]), fresh(op.result_types[2])};
        s.text = "nova.layer_norm_backward -> _mlir_ciface_nova_hip_layer_norm_backward_f32(" +
                 view_str(gy) + ", " + view_str(x) + ") -> " + view_str(s.out[0]) + ", " +
                 view_str(s.out[1]) + ", " + view_str(s.out[2]);
        for (int i = 0; i < 3 && i < (int)op.results.size(); ++i) env[op.results[i]] = s.out[i];
        plan.steps.push_back(s);
      } else if (n == "nova.linear_backward" || n == "nova.matmul_backward") {
        View go, x, w;
        if ((rc = get(op, 0, go)) || (rc = get(op, 1, x)) || (rc = get(op, 2, w)) ||
            (rc = form(op, {&go, &x, &w})))
          return rc;
        if (go.dt != x.dt || x.dt != w.dt)
          return fail(NOVA_HIP_EDTYPE, "line %d: %s operands must share a stored dtype", op.line,
                      n.c_str());
        const bool lin = n == "nova.linear_backward";
        Step s;
        s.kind = lin ? "lin_bwd" : "mm_bwd";
        s.in = {go, x, w};
        for (size_t r = 0; r < op.result_types.size(); ++r) s.out.push_back(fresh(op.result_types[r]));
        s.out_dt = op.result_types[0].dt;
        s.f32_mfma = f32_mfma && x.dt == DT_F32;
        s.text = n + " -> _mlir_ciface_nova_hip_" + (lin ? "linear" : "matmul") + "_backward(" +
                 view_str(go) + ", " + view_str(x) + ", " + view_str(w) + ") -> ";
        for (size_t r = 0; r < s.out.size(); ++r) s.text += (r ? ", " : "") + view_str(s.out[r]);
        if (s.f32_mfma) s.text += " f32=mfma";
        for (size_t r = 0; r < op.results.size() && r < s.out.size(); ++r) env[op.results[r]] = s.out[r];
        plan.steps.push_back(s);
      } else if (n == "bufferization.materialize_in_destination") {
        View src, dst;
        if ((rc = get(op, 0, src)) || (rc = get(op, 1, dst))) return rc;
        if (src.shape != dst.shape || !is_dense(src) || src.dt != dst.dt)
          return fail(NOVA_HIP_ESHAPE, "line %d: materialize_in_destination of a %s value into %s",
                      op.line, view_str(src).c_str(), view_str(dst).c_str());
        if (src.buf != dst.buf) {
          Step s;
          s.kind = "copy";
          s.in = {src};
          s.out = {dst};
          s.text = "materialize_in_destination -> hipMemcpyAsync(" + view_str(dst) + " <- " +
                   view_str(src) + ")";
          plan.steps.push_back(s);
        }
        plan.out_args.push_back(plan.bufs[dst.buf].arg);
      } else {
        return fail(NOVA_HIP_EINVAL, "line %d: op '%s' is not part of this path's op surface",
                    op.line, n.c_str());
      }
    }
    // The launches pass rank-R descriptors (GEMM 3, row ops 2, labels and
    // vectors 1, binary ops 4) and fold any leading dims into the first kept
    // one; that is only the same addressing when the folded dims are
    // contiguous over it.  Operands read as flat arrays must be dense.  A view
    // whose leading dims are permuted (a nova.transpose of batch axes) is
    // refused here rather than addressed wrongly.
    for (const Step &st : plan.steps) {
      std::vector<int> ranks;  // per input: R, or 0 for "dense"
      if (st.kind == "gemm") ranks = {3, 3, 1};
      else if (st.kind == "binary") ranks = {4, 4};
      else if (st.kind == "layer_norm") ranks = {2, 1, 1};
      else if (st.kind == "sce" || st.kind == "sce_fwd_bwd" || st.kind == "sce_bwd") ranks = {2, 1};
      else if (st.kind == "ln_bwd") ranks = {2, 2, 1, 0, 0};
      else if (st.kind == "lin_bwd" || st.kind == "mm_bwd") ranks = {2, 2, 2};
      else if (st.kind == "gather") ranks = {2, 0};
      else if (st.kind == "scatter" || st.kind == "gelu" || st.kind == "gelu_bwd" ||
               st.kind == "reduce_sum" || st.kind == "idx32")
        ranks = {0, 0};
      for (size_t i = 0; i < ranks.size() && i < st.in.size(); ++i) {
        const View &v = st.in[i];
        const bool ok = ranks[i] > 0 ? leading_dims_fold(v, ranks[i]) : is_dense(v);
        if (!ok)
          return fail(NOVA_HIP_ESTRIDE,
                      "%s: operand %zu is a view whose %s (a transpose of batch axes is not on "
                      "this path)",
                      st.text.c_str(), i,
                      ranks[i] > 0 ? "leading dims are not contiguous" : "elements are not dense");
      }
    }
    for (const std::string &r : f.rets) {
      auto it = env.find(r);
      if (it == env.end()) return fail(NOVA_HIP_EINVAL, "return of undefined value %s", r.c_str());
      if (!is_dense(it->second) || it->second.dt != it->second.logical)
        return fail(NOVA_HIP_EINVAL,
                    "returned value %s is a view (transpose / folded cast) that is never "
                    "materialised on this path",
                    r.c_str());
      plan.results.push_back(it->second);
    }
    return NOVA_HIP_SUCCESS;
  }
};

// ---- execution -----------------------------------------------------------------
template <int R>
struct Desc {
  void *allocated, *aligned;
  int64_t offset, sizes[R], strides[R];
};

template <int R>
Desc<R> desc(const View &v, const std::vector<void *> &ptr) {
  Desc<R> d;
  d.allocated = d.aligned = ptr[v.buf];
  d.offset = 0;
  const int n = (int)v.shape.size();
  for (int i = 0; i < R; ++i) {
    const int j = n - R + i;
    d.sizes[i] = j >= 0 ? v.shape[j] : 1;
    d.strides[i] = j >= 0 ? v.strides[j] : 0;
  }
  // leading dims folded into the first kept one (dense leading dims only)
  for (int j = 0; j < n - R; ++j) d.sizes[0] *= v.shape[j];
  return d;
}

int32_t run_step(const Step &s, const std::vector<void *> &ptr, hipStream_t st) {
  if (s.kind == "view") return NOVA_HIP_SUCCESS;
  if (s.kind == "zero") {
    int64_t n = 1;
    for (int64_t d : s.out[0].shape) n *= d;
    // A fill kernel, not hipMemsetAsync: a caller may capture the
    // execution in a HIP graph, where memset nodes are to be avoided.  Zero
    // bits are zero in every dtype, so an even byte count of four is filled
    // as f32 words.
    const int64_t bytes = n * dt_size(s.out[0].dt);
    if (bytes % 4 == 0) {
      NovaMemRef1D d{ptr[s.out[0].buf], ptr[s.out[0].buf], 0, {bytes / 4}, {1}};
      return _mlir_ciface_nova_hip_fill_f32(&d, 0.0f);
    }
    return hipMemsetAsync(ptr[s.out[0].buf], 0, bytes, st) == hipSuccess
               ? NOVA_HIP_SUCCESS
               : fail(NOVA_HIP_EDEVICE, "memset failed");
  }
  if (s.kind == "copy") {
    int64_t n = 1;
    for (int64_t d : s.in[0].shape) n *= d;
    return hipMemcpyAsync(ptr[s.out[0].buf], ptr[s.in[0].buf], n * dt_size(s.in[0].dt),
                          hipMemcpyDeviceToDevice, st) == hipSuccess
               ? NOVA_HIP_SUCCESS
               : fail(NOVA_HIP_EDEVICE, "device copy failed");
  }
  if (s.kind == "gemm") {
    const View &a = s.in[0], &b = s.in[1], &c = s.out[0];
    Desc<3> A = desc<3>(a, ptr), B = desc<3>(b, ptr), C = desc<3>(c, ptr);
    // rank-2 operands of a batched product broadcast over the batch
    if (a.shape.size() == 2) A.strides[0] = 0;
    if (b.shape.size() == 2) B.strides[0] = 0;
    if (a.shape.size() == 2 && c.shape.size() == 3) A.sizes[0] = 1;
    if (b.shape.size() == 2 && c.shape.size() == 3) B.sizes[0] = 1;
    Desc<1> bias;
    const Desc<1> *pb = nullptr;
    int bias_dt = 0;
    if (s.in.size() > 2) {
      bias = desc<1>(s.in[2], ptr);
      pb = &bias;
      bias_dt = s.in[2].dt;
    }
    if (a.dt != b.dt) return fail(NOVA_HIP_EDTYPE, "GEMM operands stored as %s and %s", dt_name(a.dt), dt_name(b.dt));
    return _mlir_ciface_nova_hip_gemm(reinterpret_cast<const NovaMemRef3D *>(&A),
                                      reinterpret_cast<const NovaMemRef3D *>(&B),
                                      reinterpret_cast<NovaMemRef3D *>(&C),
                                      reinterpret_cast<const NovaMemRef1D *>(pb),
                                      NOVA_HIP_GEMM_FLAGS(a.dt, s.out_dt, s.epi, bias_dt) |
                                          (s.acc_out ? NOVA_HIP_GEMM_ACC_OUT : 0) |
                                          (s.acc_c ? NOVA_HIP_GEMM_ACC_C : 0) |
                                          (s.f32_mfma ? NOVA_HIP_GEMM_F32_MFMA : 0));
  }
  if (s.kind == "layer_norm") {
    Desc<2> x = desc<2>(s.in[0], ptr), y = desc<2>(s.out[0], ptr);
    Desc<1> g = desc<1>(s.in[1], ptr), b = desc<1>(s.in[2], ptr);
    Desc<1> S = desc<1>(s.out[1], ptr), r = desc<1>(s.out[2], ptr);
    return _mlir_ciface_nova_hip_layer_norm_f32(
        reinterpret_cast<const NovaMemRef2D *>(&x), reinterpret_cast<const NovaMemRef1D *>(&g),
        reinterpret_cast<const NovaMemRef1D *>(&b), reinterpret_cast<NovaMemRef2D *>(&y),
        reinterpret_cast<NovaMemRef1D *>(&S), reinterpret_cast<NovaMemRef1D *>(&r), 1e-5f);
  }
  if (s.kind == "sce") {
    Desc<2> x = desc<2>(s.in[0], ptr);
    Desc<1> t = desc<1>(s.in[1], ptr), loss = desc<1>(s.out[1], ptr);
    Desc<2> sm;
    const bool has_sm = s.out[0].buf >= 0;
    if (has_sm) sm = desc<2>(s.out[0], ptr);
    return _mlir_ciface_nova_hip_sce_f32(reinterpret_cast<const NovaMemRef2D *>(&x),
                                         reinterpret_cast<const NovaMemRef1D *>(&t),
                                         reinterpret_cast<NovaMemRef1D *>(&loss),
                                         has_sm ? reinterpret_cast<NovaMemRef2D *>(&sm) : nullptr);
  }
  if (s.kind == "sce_fwd_bwd") {
    Desc<2> x = desc<2>(s.in[0], ptr), g = desc<2>(s.out[0], ptr);
    Desc<1> t = desc<1>(s.in[1], ptr), loss = desc<1>(s.out[1], ptr);
    return _mlir_ciface_nova_hip_sce_fwd_bwd_f32(reinterpret_cast<const NovaMemRef2D *>(&x),
                                                 reinterpret_cast<const NovaMemRef1D *>(&t),
                                                 reinterpret_cast<NovaMemRef1D *>(&loss),
                                                 reinterpret_cast<NovaMemRef2D *>(&g));
  }
  if (s.kind == "sce_bwd") {
    Desc<2> sm = desc<2>(s.in[0], ptr), g = desc<2>(s.out[0], ptr);
    Desc<1> t = desc<1>(s.in[1], ptr);
    return _mlir_ciface_nova_hip_sce_backward_f32(reinterpret_cast<const NovaMemRef2D *>(&sm),
                                                  reinterpret_cast<const NovaMemRef1D *>(&t),
                                                  reinterpret_cast<NovaMemRef2D *>(&g));
  }
  if (s.kind == "ln_bwd") {
    Desc<2> gy = desc<2>(s.in[0], ptr), x = desc<2>(s.in[1], ptr), dx = desc<2>(s.out[0], ptr);
    Desc<1> g = desc<1>(s.in[2], ptr), dg = desc<1>(s.out[1], ptr), db = desc<1>(s.out[2], ptr);
    // stats may carry a trailing unit dim ([R, 1]): fold to [R]
    View S = s.in[3], r = s.in[4];
    if (S.shape.size() >= 2 && S.shape.back() == 1) { S.shape.pop_back(); S.strides.pop_back(); }
    if (r.shape.size() >= 2 && r.shape.back() == 1) { r.shape.pop_back(); r.strides.pop_back(); }
    Desc<1> dS = desc<1>(S, ptr), dr = desc<1>(r, ptr);
    dS.strides[0] = dr.strides[0] = 1;
    return _mlir_ciface_nova_hip_layer_norm_backward_f32(
        reinterpret_cast<const NovaMemRef2D *>(&gy), reinterpret_cast<const NovaMemRef2D *>(&x),
        reinterpret_cast<const NovaMemRef1D *>(&g), reinterpret_cast<const NovaMemRef1D *>(&dS),
        reinterpret_cast<const NovaMemRef1D *>(&dr), reinterpret_cast<NovaMemRef2D *>(&dx),
        reinterpret_cast<NovaMemRef1D *>(&dg), reinterpret_cast<NovaMemRef1D *>(&db));
  }
  if (s.kind == "lin_bwd" || s.kind == "mm_bwd") {
    Desc<2> go = desc<2>(s.in[0], ptr), x = desc<2>(s.in[1], ptr), w = desc<2>(s.in[2], ptr);
    Desc<2> o0 = desc<2>(s.out[0], ptr), o1 = desc<2>(s.out[1], ptr);
    const int32_t flags = NOVA_HIP_GEMM_FLAGS(s.in[1].dt, s.out_dt, 0, 0) |
                          (s.f32_mfma ? NOVA_HIP_GEMM_F32_MFMA : 0);
    if (s.kind == "mm_bwd")
      return _mlir_ciface_nova_hip_matmul_backward(
          reinterpret_cast<const NovaMemRef2D *>(&go), reinterpret_cast<const NovaMemRef2D *>(&x),
          reinterpret_cast<const NovaMemRef2D *>(&w), reinterpret_cast<NovaMemRef2D *>(&o0),
          reinterpret_cast<NovaMemRef2D *>(&o1), flags);
    Desc<1> o2 = desc<1>(s.out[2], ptr);
    return _mlir_ciface_nova_hip_linear_backward(
        reinterpret_cast<const NovaMemRef2D *>(&go), reinterpret_cast<const NovaMemRef2D *>(&x),
        reinterpret_cast<const NovaMemRef2D *>(&w), reinterpret_cast<NovaMemRef2D *>(&o0),
        reinterpret_cast<NovaMemRef2D *>(&o1), reinterpret_cast<NovaMemRef1D *>(&o2), flags);
  }
  auto flat1 = [&](const View &v) {
    Desc<1> d;
    d.allocated = d.aligned = ptr[v.buf];
    d.offset = 0;
    d.sizes[0] = numel_of(v.shape);
    d.strides[0] = 1;
    return d;
  };
  if (s.kind == "fill") {
    Desc<1> o = flat1(s.out[0]);
    return _mlir_ciface_nova_hip_fill_f32(reinterpret_cast<NovaMemRef1D *>(&o), s.value);
  }
  if (s.kind == "binary") {
    Desc<4> a = desc<4>(s.in[0], ptr), b = desc<4>(s.in[1], ptr), c = desc<4>(s.out[0], ptr);
    return _mlir_ciface_nova_hip_binary_f32(reinterpret_cast<const NovaMemRef4D *>(&a),
                                            reinterpret_cast<const NovaMemRef4D *>(&b),
                                            reinterpret_cast<NovaMemRef4D *>(&c), s.epi);
  }
  if (s.kind == "gelu") {
    Desc<1> x = flat1(s.in[0]), y = flat1(s.out[0]);
    return _mlir_ciface_nova_hip_gelu_f32(reinterpret_cast<const NovaMemRef1D *>(&x),
                                          reinterpret_cast<NovaMemRef1D *>(&y));
  }
  if (s.kind == "gelu_bwd") {
    Desc<1> go = flat1(s.in[0]), x = flat1(s.in[1]), o = flat1(s.out[0]);
    return _mlir_ciface_nova_hip_gelu_backward_f32(reinterpret_cast<const NovaMemRef1D *>(&go),
                                                   reinterpret_cast<const NovaMemRef1D *>(&x),
                                                   reinterpret_cast<NovaMemRef1D *>(&o));
  }
  if (s.kind == "gather") {
    Desc<2> t = desc<2>(s.in[0], ptr), o = desc<2>(s.out[0], ptr);
    Desc<1> i = flat1(s.in[1]);
    return _mlir_ciface_nova_hip_gather_f32(reinterpret_cast<const NovaMemRef2D *>(&t),
                                            reinterpret_cast<const NovaMemRef1D *>(&i),
                                            reinterpret_cast<NovaMemRef2D *>(&o), s.epi);
  }
  if (s.kind == "scatter") {
    Desc<2> o = desc<2>(s.out[0], ptr);
    Desc<1> i = flat1(s.in[0]);
    Desc<2> src;
    src.allocated = src.aligned = ptr[s.in[1].buf];
    src.offset = 0;
    src.sizes[0] = numel_of(s.in[0].shape);
    src.sizes[1] = s.out[0].shape[1];
    src.strides[0] = src.sizes[1];
    src.strides[1] = 1;
    return _mlir_ciface_nova_hip_scatter_add_f32(reinterpret_cast<NovaMemRef2D *>(&o),
                                                 reinterpret_cast<const NovaMemRef1D *>(&i),
                                                 reinterpret_cast<const NovaMemRef2D *>(&src),
                                                 s.epi);
  }
  if (s.kind == "reduce_sum") {
    Desc<3> x;
    x.allocated = x.aligned = ptr[s.in[0].buf];
    x.offset = 0;
    x.sizes[0] = s.dims[0];
    x.sizes[1] = s.dims[1];
    x.sizes[2] = s.dims[2];
    x.strides[0] = s.dims[1] * s.dims[2];
    x.strides[1] = s.dims[2];
    x.strides[2] = 1;
    Desc<2> o;
    o.allocated = o.aligned = ptr[s.out[0].buf];
    o.offset = 0;
    o.sizes[0] = s.dims[0];
    o.sizes[1] = s.dims[2];
    o.strides[0] = s.dims[2];
    o.strides[1] = 1;
    return _mlir_ciface_nova_hip_reduce_sum_f32(reinterpret_cast<const NovaMemRef3D *>(&x),
                                                reinterpret_cast<NovaMemRef2D *>(&o));
  }
  if (s.kind == "idx32") {
    Desc<1> src = flat1(s.in[0]), dst = flat1(s.out[0]);
    return _mlir_ciface_nova_hip_index_to_i32(reinterpret_cast<const NovaMemRef1D *>(&src),
                                              reinterpret_cast<NovaMemRef1D *>(&dst), s.in[0].dt);
  }
  return fail(NOVA_HIP_EINVAL, "internal: unknown step %s", s.kind.c_str());
}

}  // namespace

struct NovaRunProgram {
  std::vector<Func> funcs;
  // Device buffers of each function's last execution, reused by the next one
  // when the plan's buffer sizes match (a training loop runs the same step
  // over and over); freed by nova_run_free.
  mutable std::mutex mu;
  mutable std::map<std::string, std::vector<std::pair<void *, int64_t>>> buffers;
  // Per function: an event recorded on the stream of its last device
  // execution, after that execution's last launch.  The next execution (on
  // any stream) waits for it before touching the held buffers, so two
  // executions of one program never run on those buffers at once; and the
  // buffers are freed only once it has completed.
  mutable std::map<std::string, hipEvent_t> done;
  int f32_gemm = NOVA_RUN_F32_GEMM_EXACT;  // nova_run_set_f32_gemm
  const Func *find(const char *name) const {
    for (const Func &f : funcs)
      if (name && f.name == name) return &f;
    return funcs.size() == 1 && !name ? &funcs[0] : nullptr;
  }
  void release() {
    for (auto &kv : done) {
      (void)hipEventSynchronize(kv.second);
      (void)hipEventDestroy(kv.second);
    }
    done.clear();
    for (auto &kv : buffers)
      for (auto &b : kv.second)
        if (b.first) (void)hipFree(b.first);
    buffers.clear();
  }
  ~NovaRunProgram() { release(); }
};

namespace {
int32_t plan_of(const NovaRunProgram *p, const char *func, Plan &out, const Func **fo) {
  t_err[0] = 0;
  if (!p) return fail(NOVA_HIP_EINVAL, "null program");
  const Func *f = p->find(func);
  if (!f) return fail(NOVA_HIP_EINVAL, "no function @%s", func ? func : "(null)");
  Planner pl(*f, p->f32_gemm == NOVA_RUN_F32_GEMM_MFMA);
  int32_t rc = pl.run();
  if (rc) return rc;
  out = pl.plan;
  if (fo) *fo = f;
  return NOVA_HIP_SUCCESS;
}

void fill_info(const Type &t, int32_t *dtype, int32_t *rank, int64_t *shape) {
  if (dtype) *dtype = t.dt;
  if (rank) *rank = (int32_t)t.shape.size();
  if (shape)
    for (size_t i = 0; i < t.shape.size() && i < 8; ++i) shape[i] = t.shape[i];
}
}  // namespace

extern "C" {

NovaRunProgram *nova_run_parse(const char *text_in) {
  t_err[0] = 0;
  if (!text_in) {
    fail(NOVA_HIP_EINVAL, "null text");
    return nullptr;
  }
  const std::string text = strip_comments(text_in);
  std::unique_ptr<NovaRunProgram> p(new NovaRunProgram);
  size_t at = 0;
  while ((at = text.find("func.func", at)) != std::string::npos) {
    Func f;
    size_t end = 0;
    if (parse_func(text, at, end, f)) return nullptr;
    for (const Type &t : f.arg_types)
      if (t.dt < 0) {
        fail(NOVA_HIP_EINVAL, "@%s: unsupported argument type", f.name.c_str());
        return nullptr;
      }
    p->funcs.push_back(f);
    at = end;
  }
  if (p->funcs.empty()) {
    fail(NOVA_HIP_EINVAL, "no func.func in the module");
    return nullptr;
  }
  // result types: from the values returned
  for (Func &f : p->funcs) {
    Planner pl(f);
    if (pl.run()) continue;  // reported again by plan / execute
    for (const View &v : pl.plan.results) f.ret_types.push_back(Type{v.shape, v.dt, false});
  }
  return p.release();
}

void nova_run_free(NovaRunProgram *p) { delete p; }

int32_t nova_run_set_f32_gemm(NovaRunProgram *p, int32_t mode) {
  t_err[0] = 0;
  if (!p) return fail(NOVA_HIP_EINVAL, "null program");
  if (mode != NOVA_RUN_F32_GEMM_EXACT && mode != NOVA_RUN_F32_GEMM_MFMA)
    return fail(NOVA_HIP_EINVAL, "unknown f32 GEMM mode %d", mode);
  std::lock_guard<std::mutex> lock(p->mu);
  p->f32_gemm = mode;
  return NOVA_HIP_SUCCESS;
}

const char *nova_run_last_error(void) { return t_err; }

int32_t nova_run_num_funcs(const NovaRunProgram *p) { return p ? (int32_t)p->funcs.size() : 0; }

const char *nova_run_func_name(const NovaRunProgram *p, int32_t i) {
  return p && i >= 0 && i < (int32_t)p->funcs.size() ? p->funcs[i].name.c_str() : nullptr;
}

int32_t nova_run_num_args(const NovaRunProgram *p, const char *func) {
  const Func *f = p ? p->find(func) : nullptr;
  return f ? (int32_t)f->arg_types.size() : -1;
}

int32_t nova_run_num_results(const NovaRunProgram *p, const char *func) {
  Plan pl;
  if (plan_of(p, func, pl, nullptr)) return -1;
  return (int32_t)pl.results.size();
}

int32_t nova_run_arg_info(const NovaRunProgram *p, const char *func, int32_t i, int32_t *dtype,
                          int32_t *rank, int64_t *shape) {
  const Func *f = p ? p->find(func) : nullptr;
  if (!f || i < 0 || i >= (int32_t)f->arg_types.size()) return fail(NOVA_HIP_EINVAL, "no argument %d", i);
  fill_info(f->arg_types[i], dtype, rank, shape);
  return NOVA_HIP_SUCCESS;
}

int32_t nova_run_result_info(const NovaRunProgram *p, const char *func, int32_t i,
                             int32_t *dtype, int32_t *rank, int64_t *shape) {
  Plan pl;
  int32_t rc = plan_of(p, func, pl, nullptr);
  if (rc) return rc;
  if (i < 0 || i >= (int32_t)pl.results.size()) return fail(NOVA_HIP_EINVAL, "no result %d", i);
  const View &v = pl.results[i];
  fill_info(Type{v.shape, v.dt, false}, dtype, rank, shape);
  return NOVA_HIP_SUCCESS;
}

int32_t nova_run_plan(const NovaRunProgram *p, const char *func, char *buf, size_t len) {
  Plan pl;
  const Func *f = nullptr;
  int32_t rc = plan_of(p, func, pl, &f);
  if (rc) return rc;
  std::string s = "func @" + f->name + ":\n";
  for (const Step &st : pl.steps) s += "  " + st.text + "\n";
  s += "  return";
  for (size_t i = 0; i < pl.results.size(); ++i) s += (i ? ", " : " ") + view_str(pl.results[i]);
  s += "\n";
  if (buf && len) {
    strncpy(buf, s.c_str(), len - 1);
    buf[len - 1] = 0;
  }
  return NOVA_HIP_SUCCESS;
}

int32_t nova_run_execute(const NovaRunProgram *p, const char *func, const void *const *host_args,
                         void *const *host_results) {
  Plan pl;
  const Func *f = nullptr;
  int32_t rc = plan_of(p, func, pl, &f);
  if (rc) return rc;
  if ((!host_args && !f->arg_types.empty()) || (!host_results && !pl.results.empty()))
    return fail(NOVA_HIP_EINVAL, "null argument or result array");
  hipStream_t st = static_cast<hipStream_t>(nova_hip_get_stream());
  std::lock_guard<std::mutex> lock(p->mu);
  std::vector<void *> ptr(pl.bufs.size(), nullptr);
  // Only buffers a step or a result touches get device memory.
  std::vector<bool> used(pl.bufs.size(), false);
  for (const Step &s : pl.steps) {
    for (const View &v : s.in) if (v.buf >= 0) used[v.buf] = true;
    for (const View &v : s.out) if (v.buf >= 0) used[v.buf] = true;
  }
  for (const View &v : pl.results) used[v.buf] = true;
  // The buffers of this function's previous execution, if the plan still
  // has the same sizes; otherwise a fresh set (the old one freed).
  std::vector<std::pair<void *, int64_t>> &held = p->buffers[f->name];
  bool reuse = held.size() == pl.bufs.size();
  for (size_t b = 0; reuse && b < pl.bufs.size(); ++b)
    reuse = held[b].second == (used[b] ? pl.bufs[b].bytes : 0);
  if (!reuse) {
    (void)hipStreamSynchronize(st);
    for (auto &h : held)
      if (h.first) (void)hipFree(h.first);
    held.assign(pl.bufs.size(), {nullptr, 0});
  }
  auto cleanup = [&]() {};  // buffers stay with the program
  for (size_t b = 0; b < pl.bufs.size(); ++b) {
    if (pl.bufs[b].bytes == 0 || !used[b]) continue;
    if (!held[b].first) {
      if (hipMalloc(&held[b].first, (size_t)pl.bufs[b].bytes) != hipSuccess) {
        held[b].first = nullptr;
        return fail(NOVA_HIP_ENOMEM, "hipMalloc of %lld bytes failed",
                    (long long)pl.bufs[b].bytes);
      }
      held[b].second = pl.bufs[b].bytes;
    }
    ptr[b] = held[b].first;
    if (pl.bufs[b].arg >= 0 &&
        hipMemcpyAsync(ptr[b], host_args[pl.bufs[b].arg], (size_t)pl.bufs[b].bytes,
                       hipMemcpyHostToDevice, st) != hipSuccess) {
      cleanup();
      return fail(NOVA_HIP_EDEVICE, "copy of argument %d failed", pl.bufs[b].arg);
    }
  }
  for (const Step &s : pl.steps) {
    if ((rc = run_step(s, ptr, st))) {
      const std::string why = nova_hip_last_error();
      (void)hipStreamSynchronize(st);
      cleanup();
      if (why.size()) fail(rc, "%s: %s", s.text.c_str(), why.c_str());
      return rc;
    }
  }
  for (size_t i = 0; i < pl.results.size(); ++i) {
    const View &v = pl.results[i];
    if (hipMemcpyAsync(host_results[i], ptr[v.buf], (size_t)pl.bufs[v.buf].bytes,
                       hipMemcpyDeviceToHost, st) != hipSuccess) {
      cleanup();
      return fail(NOVA_HIP_EDEVICE, "copy of result %zu failed", i);
    }
  }
  for (int a : pl.out_args) {  // writable memref arguments hold outputs
    for (size_t b = 0; b < pl.bufs.size(); ++b)
      if (pl.bufs[b].arg == a &&
          hipMemcpyAsync(const_cast<void *>(host_args[a]), ptr[b], (size_t)pl.bufs[b].bytes,
                         hipMemcpyDeviceToHost, st) != hipSuccess) {
        cleanup();
        return fail(NOVA_HIP_EDEVICE, "copy back of argument %d failed", a);
      }
  }
  const hipError_t e = hipStreamSynchronize(st);
  cleanup();
  return e == hipSuccess ? NOVA_HIP_SUCCESS : fail(NOVA_HIP_EDEVICE, "%s", hipGetErrorString(e));
}

int32_t nova_run_execute_device(const NovaRunProgram *p, const char *func,
                                void *const *dev_args, void *const *dev_results) {
  Plan pl;
  const Func *f = nullptr;
  int32_t rc = plan_of(p, func, pl, &f);
  if (rc) return rc;
  if ((!dev_args && !f->arg_types.empty()) || (!dev_results && !pl.results.empty()))
    return fail(NOVA_HIP_EINVAL, "null argument or result array");
  for (size_t i = 0; i < f->arg_types.size(); ++i)
    if (!dev_args[i] && f->arg_types[i].numel() > 0)
      return fail(NOVA_HIP_EINVAL, "argument %zu is a null pointer", i);
  for (size_t i = 0; i < pl.results.size(); ++i)
    if (!dev_results[i] && pl.bufs[pl.results[i].buf].bytes > 0)
      return fail(NOVA_HIP_EINVAL, "result %zu is a null pointer", i);
  hipStream_t st = static_cast<hipStream_t>(nova_hip_get_stream());
  std::lock_guard<std::mutex> lock(p->mu);
  const size_t nb = pl.bufs.size();
  std::vector<void *> ptr(nb, nullptr);
  std::vector<bool> used(nb, false), mine(nb, false);
  for (const Step &s : pl.steps) {
    for (const View &v : s.in) if (v.buf >= 0) used[v.buf] = true;
    for (const View &v : s.out) if (v.buf >= 0) used[v.buf] = true;
  }
  // Arguments are the caller's device memory (writable memref arguments are
  // written in place).  A result computed into a buffer of its own is
  // computed straight into the caller's result memory; a result that is an
  // argument, or a value returned twice, is copied there at the end.
  for (size_t b = 0; b < nb; ++b)
    if (pl.bufs[b].arg >= 0) ptr[b] = dev_args[pl.bufs[b].arg];
  for (size_t i = 0; i < pl.results.size(); ++i) {
    const int b = pl.results[i].buf;
    if (pl.bufs[b].arg < 0 && !ptr[b]) ptr[b] = dev_results[i];
  }
  for (size_t b = 0; b < nb; ++b) mine[b] = used[b] && !ptr[b] && pl.bufs[b].bytes > 0;
  // The program's own buffers, kept from the last device execution of this
  // function while the plan's sizes match.
  std::vector<std::pair<void *, int64_t>> &held = p->buffers[f->name + "#device"];
  hipEvent_t &done = p->done[f->name + "#device"];
  if (!done && hipEventCreateWithFlags(&done, hipEventDisableTiming) != hipSuccess) {
    done = nullptr;
    return fail(NOVA_HIP_EDEVICE, "hipEventCreate failed");
  }
  bool reuse = held.size() == nb;
  for (size_t b = 0; reuse && b < nb; ++b)
    reuse = held[b].second == (mine[b] ? pl.bufs[b].bytes : 0);
  if (!reuse) {
    // The last execution (whatever stream it ran on) may still use them.
    (void)hipEventSynchronize(done);
    for (auto &h : held)
      if (h.first) (void)hipFree(h.first);
    held.assign(nb, {nullptr, 0});
  } else if (hipStreamWaitEvent(st, done, 0) != hipSuccess) {
    return fail(NOVA_HIP_EDEVICE, "hipStreamWaitEvent failed");
  }
  for (size_t b = 0; b < nb; ++b) {
    if (!mine[b]) continue;
    if (!held[b].first) {
      if (hipMalloc(&held[b].first, (size_t)pl.bufs[b].bytes) != hipSuccess) {
        held[b].first = nullptr;
        return fail(NOVA_HIP_ENOMEM, "hipMalloc of %lld bytes failed",
                    (long long)pl.bufs[b].bytes);
      }
      held[b].second = pl.bufs[b].bytes;
    }
    ptr[b] = held[b].first;
  }
  // Whatever happens below, the event marks the end of what was queued.
  struct Mark {
    hipEvent_t ev;
    hipStream_t st;
    ~Mark() { (void)hipEventRecord(ev, st); }
  } mark{done, st};
  for (const Step &s : pl.steps) {
    if ((rc = run_step(s, ptr, st))) {
      const std::string why = nova_hip_last_error();
      if (why.size()) fail(rc, "%s: %s", s.text.c_str(), why.c_str());
      return rc;
    }
  }
  for (size_t i = 0; i < pl.results.size(); ++i) {
    const View &v = pl.results[i];
    if (ptr[v.buf] == dev_results[i] || pl.bufs[v.buf].bytes == 0) continue;
    if (hipMemcpyAsync(dev_results[i], ptr[v.buf], (size_t)pl.bufs[v.buf].bytes,
                       hipMemcpyDeviceToDevice, st) != hipSuccess)
      return fail(NOVA_HIP_EDEVICE, "copy of result %zu failed", i);
  }
  return NOVA_HIP_SUCCESS;
}

}  // extern "C"
