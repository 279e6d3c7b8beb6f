// chain_recognizer.cpp -- text-level recognition of the Matmul -> row-Softmax
// chain, the canonical decomposed emission, and the tagging stage.
//
// Stands in for the reference's canonicalize + tagging stages, which shell out
// to mlir-opt (compiler/ir/ChainCanonicalize.cpp:77-163) and then tag the
// text (compiler/ir/Tagging.cpp:50-159).  No MLIR library is involved: the
// chain has a fixed structure, so its extents, element types, softmax form and
// logit scaling are read off the text.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <regex>
#include <sstream>

#include "chain_spec.h"
#include "wtc/wtc_hip.h"

namespace wtc {

const char* elem_mlir_name(Elem e) {
  switch (e) {
    case Elem::F32: return "f32";
    case Elem::F16: return "f16";
    case Elem::BF16: return "bf16";
    case Elem::F8E4M3FN: return "f8E4M3FN";
    default: return "?";
  }
}

int elem_bytes(Elem e) {
  switch (e) {
    case Elem::F32: return 4;
    case Elem::F16:
    case Elem::BF16: return 2;
    case Elem::F8E4M3FN: return 1;
    default: return 0;
  }
}

int elem_to_dtype_code(Elem e) {
  switch (e) {
    case Elem::F32: return WTC_DTYPE_F32;
    case Elem::F16: return WTC_DTYPE_F16;
    case Elem::BF16: return WTC_DTYPE_BF16;
    case Elem::F8E4M3FN: return WTC_DTYPE_FP8_E4M3;
    default: return -1;
  }
}

static Elem parse_elem(const std::string& s) {
  if (s == "f32") return Elem::F32;
  if (s == "f16") return Elem::F16;
  if (s == "bf16") return Elem::BF16;
  if (s == "f8E4M3FN") return Elem::F8E4M3FN;
  return Elem::Unknown;
}

struct TensorType {
  std::vector<int64_t> dims;
  Elem elem = Elem::Unknown;
  std::string elem_name;
};

// "tensor<8192x64xf16>" -> dims {8192, 64}, f16.  Dynamic dims are rejected.
static bool parse_tensor(const std::string& t, TensorType& out) {
  static const std::regex re(R"(^\s*tensor<([0-9x]+)x([A-Za-z0-9]+)>\s*$)");
  std::smatch mm;
  if (!std::regex_match(t, mm, re)) return false;
  out.dims.clear();
  std::stringstream ss(mm[1].str());
  std::string d;
  while (std::getline(ss, d, 'x')) {
    if (d.empty()) return false;
    out.dims.push_back(std::stoll(d));
  }
  out.elem_name = mm[2].str();
  out.elem = parse_elem(out.elem_name);
  return true;
}

static int count_of(const std::string& text, const char* needle) {
  int c = 0;
  size_t pos = 0;
  const size_t len = std::strlen(needle);
  while ((pos = text.find(needle, pos)) != std::string::npos) {
    ++c;
    pos += len;
  }
  return c;
}

static std::string strip_comments(const std::string& text) {
  std::ostringstream o;
  std::istringstream in(text);
  std::string line;
  while (std::getline(in, line)) {
    const size_t p = line.find("//");
    o << (p == std::string::npos ? line : line.substr(0, p)) << '\n';
  }
  return o.str();
}

bool recognize_chain(const std::string& raw, ChainSpec& spec, std::string& diag) {
  const std::string text = strip_comments(raw);
  spec = ChainSpec{};
  // ---- function signature
  static const std::regex fn_re(R"(func\.func\s+@[\w$.]+\s*\(([^)]*)\)\s*->\s*\(?\s*(tensor<[^>]+>))");
  std::smatch fm;
  if (!std::regex_search(text, fm, fn_re)) {
    diag = "no func.func returning a tensor found";
    return false;
  }
  std::map<std::string, std::string> arg_types;  // %name -> type text
  {
    const std::string args = fm[1].str();
    static const std::regex arg_re(R"((%[\w]+)\s*:\s*(tensor<[^>]+>|[A-Za-z0-9]+))");
    for (std::sregex_iterator it(args.begin(), args.end(), arg_re), end; it != end; ++it)
      arg_types[(*it)[1].str()] = (*it)[2].str();
  }
  TensorType ret;
  if (!parse_tensor(fm[2].str(), ret)) {
    diag = "cannot parse result type " + fm[2].str();
    return false;
  }
  // ---- matmul
  static const std::regex mm_re(
      R"(linalg\.(batch_)?matmul\s*ins\(\s*(%[\w]+)\s*,\s*(%[\w]+)\s*:\s*(tensor<[^>]+>)\s*,\s*(tensor<[^>]+>)\s*\)\s*outs\(\s*(%[\w]+)\s*:\s*(tensor<[^>]+>)\s*\))");
  std::smatch mmm;
  if (!std::regex_search(text, mmm, mm_re)) {
    diag = "no linalg.matmul / linalg.batch_matmul with ins/outs found";
    return false;
  }
  spec.batched = mmm[1].matched;
  TensorType ta, tb, tc;
  if (!parse_tensor(mmm[4].str(), ta) || !parse_tensor(mmm[5].str(), tb) ||
      !parse_tensor(mmm[7].str(), tc)) {
    diag = "cannot parse matmul operand types";
    return false;
  }
  if (!arg_types.count(mmm[2].str()) || !arg_types.count(mmm[3].str())) {
    diag = "matmul operands must be function arguments";
    return false;
  }
  const size_t rank = spec.batched ? 3 : 2;
  if (ta.dims.size() != rank || tb.dims.size() != rank || tc.dims.size() != rank ||
      ret.dims.size() != rank) {
    diag = "operand ranks do not match the matmul kind";
    return false;
  }
  const size_t o = rank - 2;
  spec.batch = spec.batched ? ta.dims[0] : 1;
  spec.m = ta.dims[o];
  spec.k = ta.dims[o + 1];
  spec.n = tb.dims[o + 1];
  if (tb.dims[o] != spec.k || tc.dims[o] != spec.m || tc.dims[o + 1] != spec.n ||
      ret.dims[o] != spec.m || ret.dims[o + 1] != spec.n ||
      (spec.batched && (tb.dims[0] != spec.batch || tc.dims[0] != spec.batch ||
                        ret.dims[0] != spec.batch))) {
    diag = "inconsistent matmul / result extents";
    return false;
  }
  if (ta.elem != tb.elem) {
    diag = "A and B element types differ";
    return false;
  }
  spec.in = ta.elem;
  spec.acc = tc.elem;
  spec.out = ret.elem;
  if (spec.in == Elem::Unknown) {
    diag = "unsupported input element type " + ta.elem_name +
           " (f32, f16, bf16, f8E4M3FN are supported)";
    return false;
  }
  if (spec.out == Elem::Unknown || spec.out == Elem::F8E4M3FN) {
    diag = "unsupported result element type " + ret.elem_name;
    return false;
  }
  if (spec.acc == Elem::Unknown || spec.acc == Elem::F8E4M3FN) {
    diag = "unsupported matmul accumulator type " + tc.elem_name;
    return false;
  }
  // ---- softmax form
  spec.matmul_ops = count_of(text, "linalg.matmul") + count_of(text, "linalg.batch_matmul");
  spec.generic_ops = count_of(text, "linalg.generic");
  spec.reduction_hints = count_of(text, "\"reduction\"");
  spec.exp_ops = count_of(text, "math.exp");
  spec.div_ops = count_of(text, "arith.divf");
  if (text.find("linalg.softmax") != std::string::npos) {
    spec.form = SoftmaxForm::Named;
    static const std::regex dim_re(R"(linalg\.softmax\s+dimension\(\s*([0-9]+)\s*\))");
    std::smatch dm;
    if (std::regex_search(text, dm, dim_re) && std::stoll(dm[1].str()) != (int64_t)rank - 1) {
      diag = "linalg.softmax must reduce over the last dimension";
      return false;
    }
  } else {
    const bool has_max = text.find("arith.maximumf") != std::string::npos ||
                         text.find("arith.maxnumf") != std::string::npos;
    if (!has_max || spec.exp_ops == 0 || spec.div_ops == 0 || spec.reduction_hints < 2) {
      diag = "no row softmax (max / exp / sum / div generics or linalg.softmax) found";
      return false;
    }
    spec.form = SoftmaxForm::Decomposed;
  }
  // ---- logit scaling: arith.mulf by a constant or by f32 scalar arguments
  std::map<std::string, double> consts;
  static const std::regex cst_re(R"((%[\w]+)\s*=\s*arith\.constant\s+([-+0-9.eE]+)\s*:\s*f32)");
  for (std::sregex_iterator it(text.begin(), text.end(), cst_re), end; it != end; ++it)
    consts[(*it)[1].str()] = std::stod((*it)[2].str());
  static const std::regex mul_re(R"(arith\.mulf\s+(%[\w]+)\s*,\s*(%[\w]+))");
  for (std::sregex_iterator it(text.begin(), text.end(), mul_re), end; it != end; ++it) {
    for (int i = 1; i <= 2; ++i) {
      const std::string name = (*it)[i].str();
      if (consts.count(name)) spec.logit_scale *= consts[name];
      auto at = arg_types.find(name);
      if (at != arg_types.end() && at->second == "f32") spec.runtime_scales = true;
    }
  }
  if (!std::isfinite(spec.logit_scale)) {
    diag = "non-finite logit scale";
    return false;
  }
  diag.clear();
  return true;
}

// ---------------------------------------------------------------------------
// canonical decomposed emission
// ---------------------------------------------------------------------------
static std::string tensor_str(const ChainSpec& s, int64_t d1, int64_t d2, Elem e) {
  std::ostringstream o;
  o << "tensor<";
  if (s.batched) o << s.batch << "x";
  o << d1 << "x" << d2 << "x" << elem_mlir_name(e) << ">";
  return o.str();
}

static std::string fmt_double(double v) {
  char buf[64];
  std::snprintf(buf, sizeof buf, "%.9e", v);
  return buf;
}

std::string emit_canonical_mlir(const ChainSpec& s) {
  const bool b = s.batched;
  const std::string id = b ? "affine_map<(d0, d1, d2) -> (d0, d1, d2)>"
                           : "affine_map<(d0, d1) -> (d0, d1)>";
  const std::string row = b ? "affine_map<(d0, d1, d2) -> (d0, d1)>" : "affine_map<(d0, d1) -> (d0)>";
  const std::string par = b ? "\"parallel\", \"parallel\", \"parallel\"" : "\"parallel\", \"parallel\"";
  const std::string red = b ? "\"parallel\", \"parallel\", \"reduction\"" : "\"parallel\", \"reduction\"";
  const std::string ta = tensor_str(s, s.m, s.k, s.in);
  const std::string tb = tensor_str(s, s.k, s.n, s.in);
  const std::string tacc = tensor_str(s, s.m, s.n, s.acc);
  const std::string tf = tensor_str(s, s.m, s.n, Elem::F32);
  const std::string tout = tensor_str(s, s.m, s.n, s.out);
  std::ostringstream v;
  v << (b ? "tensor<" + std::to_string(s.batch) + "x" + std::to_string(s.m) + "xf32>"
          : "tensor<" + std::to_string(s.m) + "xf32>");
  const std::string tvec = v.str();
  std::ostringstream o;
  o << "// Matmul -> row-Softmax chain, canonical decomposed form (wtc canonicalize).\n";
  o << "module {\n";
  o << "  func.func @main(%A: " << ta << ", %B: " << tb;
  if (s.runtime_scales) o << ", %scale_a: f32, %scale_b: f32";
  o << ") -> " << tout << " {\n";
  o << "    %acc_zero = arith.constant 0.0 : " << elem_mlir_name(s.acc) << "\n";
  o << "    %f0 = arith.constant 0.0 : f32\n";
  o << "    %neg_inf = arith.constant -3.4028235e+38 : f32\n";
  if (s.logit_scale != 1.0) o << "    %logit_scale = arith.constant " << fmt_double(s.logit_scale) << " : f32\n";
  o << "    %c0 = tensor.empty() : " << tacc << "\n";
  o << "    %c_init = linalg.fill ins(%acc_zero : " << elem_mlir_name(s.acc) << ") outs(%c0 : " << tacc
    << ") -> " << tacc << "\n";
  o << "    %C0 = linalg." << (b ? "batch_matmul" : "matmul") << "\n";
  o << "      ins(%A, %B : " << ta << ", " << tb << ")\n";
  o << "      outs(%c_init : " << tacc << ") -> " << tacc << "\n";
  // widen (+ scale) to f32 logits
  o << "    %x0 = tensor.empty() : " << tf << "\n";
  o << "    %C = linalg.generic {indexing_maps = [" << id << ", " << id << "], iterator_types = [" << par
    << "]}\n";
  o << "      ins(%C0 : " << tacc << ") outs(%x0 : " << tf << ") {\n";
  o << "    ^bb0(%in: " << elem_mlir_name(s.acc) << ", %o: f32):\n";
  std::string cur = "%in";
  if (s.acc != Elem::F32) {
    o << "      %w = arith.extf %in : " << elem_mlir_name(s.acc) << " to f32\n";
    cur = "%w";
  }
  if (s.runtime_scales) {
    o << "      %sa = arith.mulf " << cur << ", %scale_a : f32\n";
    o << "      %sab = arith.mulf %sa, %scale_b : f32\n";
    cur = "%sab";
  }
  if (s.logit_scale != 1.0) {
    o << "      %sl = arith.mulf " << cur << ", %logit_scale : f32\n";
    cur = "%sl";
  }
  o << "      linalg.yield " << cur << " : f32\n";
  o << "    } -> " << tf << "\n";
  // max
  o << "    %max0 = tensor.empty() : " << tvec << "\n";
  o << "    %max_init = linalg.fill ins(%neg_inf : f32) outs(%max0 : " << tvec << ") -> " << tvec << "\n";
  o << "    %max = linalg.generic {indexing_maps = [" << id << ", " << row << "], iterator_types = [" << red
    << "]}\n";
  o << "      ins(%C : " << tf << ") outs(%max_init : " << tvec << ") {\n";
  o << "    ^bb0(%in: f32, %acc: f32):\n";
  o << "      %m = arith.maximumf %in, %acc : f32\n";
  o << "      linalg.yield %m : f32\n";
  o << "    } -> " << tvec << "\n";
  // exp(C - max)
  o << "    %e0 = tensor.empty() : " << tf << "\n";
  o << "    %exp_sub = linalg.generic {indexing_maps = [" << id << ", " << row << ", " << id
    << "], iterator_types = [" << par << "]}\n";
  o << "      ins(%C, %max : " << tf << ", " << tvec << ") outs(%e0 : " << tf << ") {\n";
  o << "    ^bb0(%x: f32, %mx: f32, %o: f32):\n";
  o << "      %d = arith.subf %x, %mx : f32\n";
  o << "      %e = math.exp %d : f32\n";
  o << "      linalg.yield %e : f32\n";
  o << "    } -> " << tf << "\n";
  // sum
  o << "    %s0 = tensor.empty() : " << tvec << "\n";
  o << "    %sum_init = linalg.fill ins(%f0 : f32) outs(%s0 : " << tvec << ") -> " << tvec << "\n";
  o << "    %sum = linalg.generic {indexing_maps = [" << id << ", " << row << "], iterator_types = [" << red
    << "]}\n";
  o << "      ins(%exp_sub : " << tf << ") outs(%sum_init : " << tvec << ") {\n";
  o << "    ^bb0(%in: f32, %acc: f32):\n";
  o << "      %r = arith.addf %in, %acc : f32\n";
  o << "      linalg.yield %r : f32\n";
  o << "    } -> " << tvec << "\n";
  // div (+ narrowing)
  o << "    %y0 = tensor.empty() : " << tout << "\n";
  o << "    %out = linalg.generic {indexing_maps = [" << id << ", " << row << ", " << id
    << "], iterator_types = [" << par << "]}\n";
  o << "      ins(%exp_sub, %sum : " << tf << ", " << tvec << ") outs(%y0 : " << tout << ") {\n";
  o << "    ^bb0(%e: f32, %s: f32, %o: " << elem_mlir_name(s.out) << "):\n";
  o << "      %y = arith.divf %e, %s : f32\n";
  if (s.out != Elem::F32) {
    o << "      %yt = arith.truncf %y : f32 to " << elem_mlir_name(s.out) << "\n";
    o << "      linalg.yield %yt : " << elem_mlir_name(s.out) << "\n";
  } else {
    o << "      linalg.yield %y : f32\n";
  }
  o << "    } -> " << tout << "\n";
  o << "    return %out : " << tout << "\n";
  o << "  }\n";
  o << "}\n";
  return o.str();
}

// ---------------------------------------------------------------------------
// tagging (same comment tags and JSON keys as compiler/ir/Tagging.cpp:94-150)
// ---------------------------------------------------------------------------
static std::string json_escape(const std::string& s) {
  std::string o;
  for (char c : s) {
    if (c == '"' || c == '\\') o += '\\';
    o += c;
  }
  return o;
}

void tag_chain(const std::string& text, const ChainSpec& spec, const std::string& source,
               std::string& tagged_mlir, std::string& tags_json) {
  std::ostringstream t;
  t << "// [wtc tagging] tags are emitted as comments for readability\n";
  bool mm = false, red = false, ex = false, dv = false;
  std::istringstream in(text);
  std::string line;
  while (std::getline(in, line)) {
    if (!mm && (line.find("linalg.matmul") != std::string::npos ||
                line.find("linalg.batch_matmul") != std::string::npos)) {
      t << "// wtc.tag: welder.matmul_anchor\n";
      mm = true;
    }
    if (!red && line.find("\"reduction\"") != std::string::npos) {
      t << "// wtc.tag: welder.row_reduction\n";
      red = true;
    }
    if (!ex && line.find("math.exp") != std::string::npos) {
      t << "// wtc.tag: welder.elementwise_exp\n";
      ex = true;
    }
    if (!dv && line.find("arith.divf") != std::string::npos) {
      t << "// wtc.tag: welder.elementwise_div\n";
      dv = true;
    }
    t << line << '\n';
  }
  tagged_mlir = t.str();
  std::ostringstream j;
  j << "{\n"
    << "  \"pipeline\": \"typical_chain\",\n"
    << "  \"source\": \"" << json_escape(source) << "\",\n"
    << "  \"counts\": {\n"
    << "    \"matmul\": " << count_of(text, "linalg.matmul") + count_of(text, "linalg.batch_matmul") << ",\n"
    << "    \"generic\": " << count_of(text, "linalg.generic") << ",\n"
    << "    \"reduction_hints\": " << count_of(text, "\"reduction\"") << ",\n"
    << "    \"exp\": " << count_of(text, "math.exp") << ",\n"
    << "    \"div\": " << count_of(text, "arith.divf") << "\n"
    << "  },\n"
    << "  \"problem\": {\"batch\": " << spec.batch << ", \"m\": " << spec.m << ", \"n\": " << spec.n
    << ", \"k\": " << spec.k << ", \"in\": \"" << elem_mlir_name(spec.in) << "\", \"acc\": \""
    << elem_mlir_name(spec.acc) << "\", \"out\": \"" << elem_mlir_name(spec.out) << "\"},\n"
    << "  \"tags\": [\n"
    << "    \"welder.matmul_anchor\",\n"
    << "    \"welder.row_reduction\",\n"
    << "    \"welder.elementwise_exp\",\n"
    << "    \"welder.elementwise_div\"\n"
    << "  ]\n"
    << "}\n";
  tags_json = j.str();
}

// ---------------------------------------------------------------------------
// files
// ---------------------------------------------------------------------------
bool read_file(const std::string& path, std::string& out) {
  std::ifstream f(path, std::ios::binary);
  if (!f) return false;
  std::ostringstream ss;
  ss << f.rdbuf();
  out = ss.str();
  return true;
}

bool write_file(const std::string& path, const std::string& text) {
  std::ofstream f(path, std::ios::binary | std::ios::trunc);
  if (!f) return false;
  f << text;
  return static_cast<bool>(f);
}

// Clears, then fills the caller's buffer with a NUL-terminated, truncated
// message (driver/WelderCompileCAPI.cpp:10-16).
void set_error(char* buf, size_t size, const std::string& msg) {
  if (!buf || size == 0) return;
  const size_t n = std::min(size - 1, msg.size());
  std::memcpy(buf, msg.data(), n);
  buf[n] = '\0';
}

}  // namespace wtc
