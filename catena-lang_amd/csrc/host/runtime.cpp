// Runtime mirror: Runtime::from_sources / exec / mem_* and Value, over a
// table of native program lowerings.
//
// Reference: catena-lang/src/runtime/runtime.rs:104-247 (API, validation
// order), catena-lang/src/runtime/value.rs:5-49 (Value / ValueKind),
// catena-lang/src/runtime/signature.rs:18-72 (name -> symbol + kinds).
// The reference compiles every source program to generated C++; this build
// has no front end (out of scope) and instead binds source programs BY NAME
// to native lowerings, checking the kinds of the declared type against the
// lowering's signature.  The stdlib programs on and around the hot path
// (nn.softmax, math.exp-approx, math.sqrt, nn.sigmoid, nn.silu,
// math.sin-approx(-full), math.cos-approx, nn.rmsnorm, tensor.*, sum-f32,
// mean-f32, max-f32) and this build's new programs are built in; user sources declare
// the rest (e.g. matmul-2x2-via-mem, sum-u64, dot-u64).
#include <cctype>
#include <cstring>
#include <new>
#include <memory>
#include <string>
#include <vector>

#include "internal.h"

using namespace catena;

namespace {

using Kind = catena_value_kind_t;
constexpr Kind kMem = CATENA_VALUE_MEM, kU64 = CATENA_VALUE_U64, kF32 = CATENA_VALUE_F32;

typedef void (*Invoke)(const catena_value_t* in, catena_value_t* out);

struct Lowering {
  const char* name;
  bool builtin;  // part of the built-in stdlib (no declaration needed)
  std::vector<Kind> inputs, outputs;
  Invoke invoke;
};

catena_value_t mem_value(catena_mem_t m) {
  catena_value_t v;
  v.kind = kMem;
  v.as.mem = m;
  return v;
}

void inv_matmul(const catena_value_t* in, catena_value_t* out) {
  catena_mem_t r;
  program_matmul_2x2_via_mem(in[0].as.mem, in[1].as.mem, in[2].as.u64, in[3].as.u64, in[4].as.u64,
                             in[5].as.u64, in[6].as.u64, in[7].as.u64, &r);
  out[0] = mem_value(r);
}
void inv_right_id(const catena_value_t* in, catena_value_t* out) {
  catena_mem_t r;
  program_matmul_right_identity_2x2_via_mem(in[0].as.mem, in[1].as.u64, in[2].as.u64, &r);
  out[0] = mem_value(r);
}
void inv_left_id(const catena_value_t* in, catena_value_t* out) {
  catena_mem_t r;
  program_matmul_left_identity_2x2_via_mem(in[0].as.mem, in[1].as.u64, in[2].as.u64, &r);
  out[0] = mem_value(r);
}
void inv_softmax(const catena_value_t* in, catena_value_t* out) {
  catena_mem_t r;
  program_nn_softmax(in[0].as.mem, &r);
  out[0] = mem_value(r);
}
void inv_exp(const catena_value_t* in, catena_value_t* out) {
  float r;
  program_math_exp_approx(in[0].as.f32, &r);
  out[0].kind = kF32;
  out[0].as.f32 = r;
}
template <void (*Program)(float, float*)>
void inv_scalar(const catena_value_t* in, catena_value_t* out) {
  float r;
  Program(in[0].as.f32, &r);
  out[0].kind = kF32;
  out[0].as.f32 = r;
}
void inv_bf16_matmul(const catena_value_t* in, catena_value_t* out) {
  catena_mem_t r;
  program_bf16_matmul_via_mem(in[0].as.mem, in[1].as.mem, in[2].as.u64, in[3].as.u64, in[4].as.u64,
                              in[5].as.u64, in[6].as.u64, in[7].as.u64, &r);
  out[0] = mem_value(r);
}
void inv_attn(const catena_value_t* in, catena_value_t* out) {
  catena_mem_t r;
  program_attn_decode_via_mem(in[0].as.mem, in[1].as.mem, in[2].as.mem, in[3].as.mem, in[4].as.u64,
                              in[5].as.u64, in[6].as.u64, in[7].as.u64, in[8].as.f32, &r);
  out[0] = mem_value(r);
}

void inv_rmsnorm(const catena_value_t* in, catena_value_t* out) {
  catena_mem_t r;
  program_nn_rmsnorm(in[0].as.mem, &r);
  out[0] = mem_value(r);
}
void inv_argmax(const catena_value_t* in, catena_value_t* out) {
  uint64_t r;
  program_tensor_argmax_f32(in[0].as.mem, &r);
  out[0].kind = kU64;
  out[0].as.u64 = r;
}

void inv_broadcast(const catena_value_t* in, catena_value_t* out) {
  catena_mem_t r;
  program_tensor_broadcast_f32(in[0].as.f32, in[1].as.u64, &r);
  out[0] = mem_value(r);
}
void inv_arange(const catena_value_t* in, catena_value_t* out) {
  catena_mem_t r;
  program_tensor_arange_f32(in[0].as.u64, &r);
  out[0] = mem_value(r);
}
void inv_slice(const catena_value_t* in, catena_value_t* out) {
  catena_mem_t r;
  program_tensor_slice_f32(in[0].as.mem, in[1].as.u64, in[2].as.u64, &r);
  out[0] = mem_value(r);
}
void inv_concat(const catena_value_t* in, catena_value_t* out) {
  catena_mem_t r;
  program_tensor_concat_f32(in[0].as.mem, in[1].as.mem, &r);
  out[0] = mem_value(r);
}
void set_f32(catena_value_t* out, float v) {
  out[0].kind = kF32;
  out[0].as.f32 = v;
}
void set_u64(catena_value_t* out, uint64_t v) {
  out[0].kind = kU64;
  out[0].as.u64 = v;
}
void inv_sum_f32(const catena_value_t* in, catena_value_t* out) {
  float r;
  program_sum_f32(in[0].as.mem, &r);
  set_f32(out, r);
}
void inv_mean_f32(const catena_value_t* in, catena_value_t* out) {
  float r;
  program_mean_f32(in[0].as.mem, &r);
  set_f32(out, r);
}
void inv_max_f32(const catena_value_t* in, catena_value_t* out) {
  float r;
  program_max_f32(in[0].as.mem, &r);
  set_f32(out, r);
}
void inv_sum_u64(const catena_value_t* in, catena_value_t* out) {
  uint64_t r;
  program_sum_u64(in[0].as.mem, &r);
  set_u64(out, r);
}
void inv_dot_u64(const catena_value_t* in, catena_value_t* out) {
  uint64_t r;
  program_dot_u64(in[0].as.mem, in[1].as.mem, &r);
  set_u64(out, r);
}

const std::vector<Lowering>& lowerings() {
  static const std::vector<Lowering> t = {
      {"matmul-2x2-via-mem", false, {kMem, kMem, kU64, kU64, kU64, kU64, kU64, kU64}, {kMem},
       inv_matmul},
      {"matmul-right-identity-2x2-via-mem", false, {kMem, kU64, kU64}, {kMem}, inv_right_id},
      {"matmul-left-identity-2x2-via-mem", false, {kMem, kU64, kU64}, {kMem}, inv_left_id},
      {"nn.softmax", true, {kMem}, {kMem}, inv_softmax},
      {"math.exp-approx", true, {kF32}, {kF32}, inv_exp},
      {"math.sqrt", true, {kF32}, {kF32}, inv_scalar<program_math_sqrt>},
      {"nn.sigmoid", true, {kF32}, {kF32}, inv_scalar<program_nn_sigmoid>},
      {"nn.silu", true, {kF32}, {kF32}, inv_scalar<program_nn_silu>},
      {"math.sin-approx", true, {kF32}, {kF32}, inv_scalar<program_math_sin_approx>},
      {"math.cos-approx", true, {kF32}, {kF32}, inv_scalar<program_math_cos_approx>},
      {"math.sin-approx-full", true, {kF32}, {kF32}, inv_scalar<program_math_sin_approx_full>},
      {"nn.rmsnorm", true, {kMem}, {kMem}, inv_rmsnorm},
      {"tensor.argmax-f32", true, {kMem}, {kU64}, inv_argmax},
      {"tensor.broadcast-f32", true, {kF32, kU64}, {kMem}, inv_broadcast},
      {"tensor.arange-f32", true, {kU64}, {kMem}, inv_arange},
      {"tensor.slice-f32", true, {kMem, kU64, kU64}, {kMem}, inv_slice},
      {"tensor.concat-f32", true, {kMem, kMem}, {kMem}, inv_concat},
      {"sum-f32", true, {kMem}, {kF32}, inv_sum_f32},
      {"mean-f32", true, {kMem}, {kF32}, inv_mean_f32},
      {"max-f32", true, {kMem}, {kF32}, inv_max_f32},
      {"sum-u64", false, {kMem}, {kU64}, inv_sum_u64},
      {"dot-u64", false, {kMem, kMem}, {kU64}, inv_dot_u64},
      {"bf16.matmul.row-major.via-mem", true,
       {kMem, kMem, kU64, kU64, kU64, kU64, kU64, kU64}, {kMem}, inv_bf16_matmul},
      {"attn.decode.via-mem", true, {kMem, kMem, kMem, kMem, kU64, kU64, kU64, kU64, kF32}, {kMem},
       inv_attn},
  };
  return t;
}

// ---------------------------------------------------------------- hexpr scan
// A minimal reader: atoms, (), [], {} and '#' line comments.  Enough to find
// `(def program NAME : TYPE = BODY)` forms and classify TYPE's components.
struct Node {
  char open = 0;  // 0 for an atom
  std::string atom;
  std::vector<Node> kids;
};

struct Reader {
  static constexpr int kMaxDepth = 4096;  // nesting bound (the reader recurses)
  const char* s;
  size_t i = 0, n;
  int depth = 0;
  std::string err;
  explicit Reader(const char* src) : s(src), n(strlen(src)) {}
  void skip() {
    while (i < n) {
      if (isspace((unsigned char)s[i])) {
        ++i;
      } else if (s[i] == '#') {
        while (i < n && s[i] != '\n') ++i;
      } else {
        break;
      }
    }
  }
  static char closer(char o) { return o == '(' ? ')' : o == '[' ? ']' : '}'; }
  bool read(Node& out) {
    skip();
    if (i >= n) return false;
    char c = s[i];
    if (c == '(' || c == '[' || c == '{') {
      if (depth >= kMaxDepth) {
        err = "brackets nested too deeply";
        return false;
      }
      ++i;
      out.open = c;
      for (;;) {
        skip();
        if (i >= n) {
          err = "unbalanced bracket";
          return false;
        }
        if (s[i] == closer(c)) {
          ++i;
          return true;
        }
        if (s[i] == ')' || s[i] == ']' || s[i] == '}') {
          err = "mismatched bracket";
          return false;
        }
        Node k;
        ++depth;
        const bool ok = read(k);
        --depth;
        if (!ok) {
          if (err.empty()) err = "unexpected end";
          return false;
        }
        out.kids.push_back(std::move(k));
      }
    }
    if (c == ')' || c == ']' || c == '}') {
      err = "unexpected closing bracket";
      return false;
    }
    size_t b = i;
    while (i < n && !isspace((unsigned char)s[i]) && !strchr("()[]{}#", s[i])) ++i;
    out.atom.assign(s + b, i - b);
    return true;
  }
};

void atoms(const Node& nd, std::vector<std::string>& acc) {
  if (!nd.open) {
    acc.push_back(nd.atom);
    return;
  }
  for (const Node& k : nd.kids) atoms(k, acc);
}

// Classify one boundary component: (cap.ref mem) -> Mem, (f32 val) -> F32,
// ({[.n] u64} :) -> U64, ...; -1 when it is not a runtime value.
int classify_one(const Node& nd) {
  std::vector<std::string> a;
  atoms(nd, a);
  auto has = [&](const char* w) {
    for (auto& x : a)
      if (x == w) return true;
    return false;
  };
  if (has("mem")) return kMem;
  if (has("f32")) return kF32;
  if (has("u64")) return kU64;
  if (has("u32")) return CATENA_VALUE_U32;
  if (has("bool")) return CATENA_VALUE_BOOL;
  return -1;
}

// One side of `IN -> OUT`: strip a `([binders.] X)` wrapper, then a brace
// list is a product of components.
bool classify_side(const std::vector<Node>& parts, std::vector<Kind>& kinds) {
  if (parts.size() != 1) return false;
  const Node* nd = &parts[0];
  if (nd->open == '(' && nd->kids.size() == 2 && nd->kids[0].open == '[') nd = &nd->kids[1];
  if (nd->open == '{') {
    for (const Node& k : nd->kids) {
      int c = classify_one(k);
      if (c < 0) return false;
      kinds.push_back((Kind)c);
    }
    return true;
  }
  int c = classify_one(*nd);
  if (c < 0) return false;
  kinds.push_back((Kind)c);
  return true;
}

struct Declared {
  std::string name;
  bool typed = false;
  std::vector<Kind> inputs, outputs;
};

void collect_defs(const Node& nd, std::vector<Declared>& out) {
  if (!nd.open) return;
  if (nd.open == '(' && nd.kids.size() >= 4 && !nd.kids[0].open && nd.kids[0].atom == "def" &&
      !nd.kids[1].open && nd.kids[1].atom == "program" && !nd.kids[2].open &&
      !nd.kids[3].open && nd.kids[3].atom == ":") {
    Declared d;
    d.name = nd.kids[2].atom;
    std::vector<Node> in, outp;
    bool arrow = false, ok = true;
    size_t j = 4;
    for (; j < nd.kids.size(); ++j) {
      const Node& k = nd.kids[j];
      if (!k.open && k.atom == "=") break;
      if (!k.open && k.atom == "->") {
        arrow = true;
        continue;
      }
      (arrow ? outp : in).push_back(k);
    }
    if (arrow) ok = classify_side(in, d.inputs) && classify_side(outp, d.outputs);
    d.typed = arrow && ok;
    out.push_back(std::move(d));
    return;
  }
  for (const Node& k : nd.kids) collect_defs(k, out);
}

struct Program {
  const Lowering* lowering;
};

struct ErrDetail {
  int64_t index = -1, expected = -1, actual = -1;
};
thread_local ErrDetail g_detail;

int exec_fail(int status, int64_t index, int64_t expected, int64_t actual, const char* fmt,
              const char* name) {
  g_detail.index = index;
  g_detail.expected = expected;
  g_detail.actual = actual;
  return fail(status, fmt, name);
}

}  // namespace

struct catena_runtime {
  std::vector<std::pair<std::string, Program>> programs;
  const Program* find(const char* name) const {
    for (auto& p : programs)
      if (p.first == name) return &p.second;
    return nullptr;
  }
};

extern "C" {

namespace {
int from_sources(const char* const* sources, size_t n_sources, const char* dialect,
                 catena_runtime_t** out);
}

int catena_runtime_from_sources(const char* const* sources, size_t n_sources, const char* dialect,
                                catena_runtime_t** out) {
  if (!out) return fail(CATENA_EXEC_BAD_CALL, "out is NULL");
  *out = nullptr;
  if (n_sources > 0 && !sources) return fail(CATENA_EXEC_BAD_CALL, "sources is NULL");
  try {
    return from_sources(sources, n_sources, dialect, out);
  } catch (const std::bad_alloc&) {
    return fail(CATENA_INIT_HOST_MEMORY, "out of host memory while reading sources");
  }
}

}  // extern "C"

namespace {
int from_sources(const char* const* sources, size_t n_sources, const char* dialect,
                 catena_runtime_t** out) {
  // GpuDialect (catena-lang/src/codegen/mod.rs:50-54): only Hip is served.
  if (!dialect || strcmp(dialect, "hip") != 0)
    return fail(CATENA_INIT_DIALECT, "GPU dialect `%s` is not supported; expected `hip`",
                dialect ? dialect : "(null)");
  std::vector<Declared> decls;
  for (size_t s = 0; s < n_sources; ++s) {
    if (!sources[s]) continue;
    Reader r(sources[s]);
    for (;;) {
      Node nd;
      if (!r.read(nd)) {
        if (!r.err.empty())
          return fail(CATENA_INIT_PARSE, "Failed to parse program: source %zu: %s at byte %zu", s,
                      r.err.c_str(), r.i);
        break;
      }
      collect_defs(nd, decls);
    }
  }
  auto rt = std::make_unique<catena_runtime>();
  for (const Lowering& l : lowerings()) {
    const Declared* d = nullptr;
    for (const Declared& x : decls)
      if (x.name == l.name) d = &x;
    if (d) {
      if (!d->typed || d->inputs != l.inputs || d->outputs != l.outputs)
        return fail(CATENA_INIT_SIGNATURE_MISMATCH,
                    "program `%s`: declared type does not match its native lowering", l.name);
    } else if (!l.builtin) {
      continue;
    }
    rt->programs.push_back({l.name, Program{&l}});
  }
  // The device is opened lazily by the first allocation or program call, so
  // parsing and exec-time validation work (and are tested) without a GPU.
  *out = rt.release();
  return CATENA_OK;
}
}  // namespace

extern "C" {

void catena_runtime_destroy(catena_runtime_t* rt) { delete rt; }

int catena_runtime_exec(catena_runtime_t* rt, const char* name, const catena_value_t* args,
                        size_t n_args, catena_value_t* outs, size_t n_outs) {
  g_detail = ErrDetail{};
  if (!rt || !name) return fail(CATENA_EXEC_BAD_CALL, "null runtime or name");
  const Program* p = rt->find(name);
  if (!p)
    return exec_fail(CATENA_EXEC_UNKNOWN_SOURCE_FUNCTION, -1, -1, -1,
                     "Unknown source function '%s'", name);
  const Lowering& l = *p->lowering;
  if (l.inputs.size() != n_args)
    return exec_fail(CATENA_EXEC_INPUT_ARITY_MISMATCH, -1, (int64_t)l.inputs.size(),
                     (int64_t)n_args, "Function '%s' input arity mismatch", name);
  if (l.outputs.size() != n_outs)
    return exec_fail(CATENA_EXEC_OUTPUT_ARITY_MISMATCH, -1, (int64_t)l.outputs.size(),
                     (int64_t)n_outs, "Function '%s' output arity mismatch", name);
  if ((n_args > 0 && !args) || (n_outs > 0 && !outs))
    return fail(CATENA_EXEC_BAD_CALL, "null argument or output array");
  for (size_t i = 0; i < n_args; ++i)
    if (args[i].kind != l.inputs[i])
      return exec_fail(CATENA_EXEC_TYPE_MISMATCH, (int64_t)i, (int64_t)l.inputs[i],
                       (int64_t)args[i].kind, "Function '%s' argument kind mismatch", name);
  // zeroed output slots (catena-lang/src/runtime/runtime.rs:238-246)
  for (size_t i = 0; i < n_outs; ++i) {
    memset(&outs[i], 0, sizeof(catena_value_t));
    outs[i].kind = l.outputs[i];
  }
  l.invoke(args, outs);
  return CATENA_EXEC_OK;
}

int catena_runtime_last_error_detail(int64_t* index, int64_t* expected, int64_t* actual) {
  if (index) *index = g_detail.index;
  if (expected) *expected = g_detail.expected;
  if (actual) *actual = g_detail.actual;
  return CATENA_OK;
}

size_t catena_runtime_program_count(const catena_runtime_t* rt) {
  return rt ? rt->programs.size() : 0;
}

const char* catena_runtime_program_name(const catena_runtime_t* rt, size_t i) {
  if (!rt || i >= rt->programs.size()) return nullptr;
  return rt->programs[i].first.c_str();
}

int catena_runtime_mem_u64(catena_runtime_t* rt, const uint64_t* values, size_t n,
                           catena_value_t* out) {
  (void)rt;
  if (!out) return fail(CATENA_ERR_INVALID_ARGUMENT, "out is NULL");
  catena_mem_t m;
  int st = catena_mem_alloc(n * 8, &m);
  if (st) return st;
  st = catena_mem_write(m, 0, values, n * 8);
  if (st) {
    catena_mem_free(&m);
    return st;
  }
  *out = mem_value(m);
  return CATENA_OK;
}

int catena_runtime_mem_f32(catena_runtime_t* rt, const float* values, size_t n,
                           catena_value_t* out) {
  (void)rt;
  if (!out) return fail(CATENA_ERR_INVALID_ARGUMENT, "out is NULL");
  catena_mem_t m;
  int st = catena_mem_alloc(n * 4, &m);
  if (st) return st;
  st = catena_mem_write(m, 0, values, n * 4);
  if (st) {
    catena_mem_free(&m);
    return st;
  }
  *out = mem_value(m);
  return CATENA_OK;
}

}  // extern "C"
