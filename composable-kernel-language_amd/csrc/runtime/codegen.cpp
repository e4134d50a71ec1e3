#include "codegen.h"

#include <hip/hiprtc.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <sstream>
#include <unordered_map>

namespace ckl::rt {

namespace {

std::string cType(const Type &t) {
  switch (t.kind) {
  case Type::F32: return "float";
  case Type::F64: return "double";
  case Type::I1: return "bool";
  case Type::I8: return "signed char";
  case Type::I32: return "int";
  case Type::I64: case Type::Index: return "long long";
  case Type::MemRef: return cType(Type::scalar(t.element)) + "*";
  default: throw CompileError("device code generation does not support type " + t.str());
  }
}

std::string unsignedType(const Type &t) {
  switch (t.kind) {
  case Type::I32: return "unsigned int";
  case Type::I64: case Type::Index: return "unsigned long long";
  case Type::I8: return "unsigned char";
  case Type::I1: return "bool";
  default: throw CompileError("integer operation on non-integer type " + t.str());
  }
}

std::string literal(const Attr &a) {
  char buf[64];
  if (a.kind == Attr::Float) {
    if (a.type.kind == Type::F32) {
      std::snprintf(buf, sizeof buf, "%af", double(float(a.f)));
    } else std::snprintf(buf, sizeof buf, "%a", a.f);
    if (std::isnan(a.f)) return a.type.kind == Type::F32 ? "__builtin_nanf(\"\")" : "__builtin_nan(\"\")";
    if (std::isinf(a.f)) return std::string(a.f < 0 ? "-" : "") + (a.type.kind == Type::F32 ? "__builtin_inff()" : "__builtin_inf()");
    return std::string("(") + buf + ")";
  }
  if (a.kind == Attr::Int) {
    if (a.type.kind == Type::I1) return a.i ? "true" : "false";
    if (a.type.kind == Type::I32) return "((int)" + std::to_string(int32_t(a.i)) + ")";
    if (a.i == INT64_MIN) return "((long long)(-9223372036854775807LL - 1))";
    return "((long long)" + std::to_string(a.i) + "LL)";
  }
  if (a.kind == Attr::Bool) return a.i ? "true" : "false";
  throw CompileError("unsupported constant in device code");
}

class KernelEmitter {
public:
  KernelEmitter(const Op &function, std::ostringstream &out) : function(function), out(out) {}

  void emit() {
    std::string symbol = function.symName();
    Block *entry = function.entry();
    out << "struct __attribute__((aligned(8))) " << symbol << "_args {\n";
    for (size_t k = 0; k < entry->args.size(); ++k) out << "  " << cType(entry->args[k]->type) << " a" << k << ";\n";
    if (entry->args.empty()) out << "  long long unused;\n";
    out << "};\n";
    out << "extern \"C\" __global__ void " << symbol << "(const " << symbol << "_args args) {\n";
    for (size_t k = 0; k < entry->args.size(); ++k) {
      std::string n = bind(entry->args[k].get());
      out << "  " << cType(entry->args[k]->type) << " " << n << " = args.a" << k << ";\n";
    }
    for (auto &op : entry->ops) statement(*op, 1);
    out << "}\n\n";
  }

private:
  const Op &function;
  std::ostringstream &out;
  std::unordered_map<const Value *, std::string> names;
  unsigned next = 0;
  std::vector<std::vector<std::string>> yieldTargets;

  std::string bind(const Value *v) {
    std::string n = "v" + std::to_string(next++);
    names[v] = n;
    return n;
  }
  std::string ref(const Value *v) {
    auto it = names.find(v);
    if (it == names.end()) throw CompileError("device code generation found an unbound value");
    return it->second;
  }
  std::string pad(int indent) { return std::string(indent * 2, ' '); }

  std::string element(const Op &op, size_t resourceIndex, size_t firstIndex) {
    const Value *buffer = op.operands[resourceIndex];
    const Type &t = buffer->type;
    if (!t.hasStaticShape()) throw CompileError("device code generation requires static buffer shapes");
    if (op.operands.size() - firstIndex != t.shape.size()) throw CompileError("indexed access rank mismatch");
    std::string linear;
    for (size_t axis = 0; axis < t.shape.size(); ++axis) {
      std::string i = "(" + ref(op.operands[firstIndex + axis]) + ")";
      linear = axis == 0 ? i : "(" + linear + ") * " + std::to_string(t.shape[axis]) + "LL + " + i;
    }
    if (linear.empty()) linear = "0";
    return ref(buffer) + "[" + linear + "]";
  }

  std::string compare(const Op &op) {
    const Attr *p = op.attr("predicate");
    if (!p) throw CompileError("comparison without predicate");
    std::string a = ref(op.operands[0]), b = ref(op.operands[1]);
    const Type &t = op.operands[0]->type;
    if (op.name == "arith.cmpi") {
      std::string u = unsignedType(t);
      std::string ua = "((" + u + ")" + a + ")", ub = "((" + u + ")" + b + ")";
      static const char *ops[] = {"==", "!=", "<", "<=", ">", ">="};
      int64_t k = p->i;
      if (k >= 0 && k <= 5) return "(" + a + " " + ops[k] + " " + b + ")";
      static const char *uops[] = {"<", "<=", ">", ">="};
      if (k >= 6 && k <= 9) return "(" + ua + " " + uops[k - 6] + " " + ub + ")";
      throw CompileError("unsupported integer predicate");
    }
    std::string nan = "(__builtin_isnan(" + a + ") || __builtin_isnan(" + b + "))";
    switch (p->i) {
    case 0: return "false";
    case 1: return "(" + a + " == " + b + ")";
    case 2: return "(" + a + " > " + b + ")";
    case 3: return "(" + a + " >= " + b + ")";
    case 4: return "(" + a + " < " + b + ")";
    case 5: return "(" + a + " <= " + b + ")";
    case 6: return "(" + a + " < " + b + " || " + a + " > " + b + ")";
    case 7: return "(!" + nan + ")";
    case 8: return "(" + a + " == " + b + " || " + nan + ")";
    case 9: return "(!(" + a + " <= " + b + "))";
    case 10: return "(!(" + a + " < " + b + "))";
    case 11: return "(!(" + a + " >= " + b + "))";
    case 12: return "(!(" + a + " > " + b + "))";
    case 13: return "(" + a + " != " + b + ")";
    case 14: return nan;
    case 15: return "true";
    }
    throw CompileError("unsupported float predicate");
  }

  std::string expression(const Op &op) {
    const std::string &n = op.name;
    auto arg = [&](size_t k) { return ref(op.operands.at(k)); };
    const Type &rt = op.results.empty() ? op.operands[0]->type : op.results[0]->type;
    if (n == "arith.constant") return literal(*op.attr("value"));
    if (n == "ckl.global_id" || n == "ckl.thread_id" || n == "ckl.block_id" || n == "ckl.block_dim" || n == "ckl.grid_dim") {
      const char *axes[] = {"x", "y", "z"};
      const Attr *axis = op.attr("axis");
      if (!axis || axis->i < 0 || axis->i > 2) throw CompileError("device coordinate requires axis 0, 1 or 2");
      std::string a = axes[axis->i];
      if (n == "ckl.global_id") return "((long long)blockIdx." + a + " * (long long)blockDim." + a + " + (long long)threadIdx." + a + ")";
      if (n == "ckl.thread_id") return "((long long)threadIdx." + a + ")";
      if (n == "ckl.block_id") return "((long long)blockIdx." + a + ")";
      if (n == "ckl.block_dim") return "((long long)blockDim." + a + ")";
      return "((long long)gridDim." + a + ")";
    }
    if (n == "arith.addf") return arg(0) + " + " + arg(1);
    if (n == "arith.subf") return arg(0) + " - " + arg(1);
    if (n == "arith.mulf") return arg(0) + " * " + arg(1);
    if (n == "arith.divf") return arg(0) + " / " + arg(1);
    if (n == "arith.negf") return "-" + arg(0);
    if (n == "arith.addi" || n == "arith.subi" || n == "arith.muli") {
      std::string u = unsignedType(rt);
      const char *o = n == "arith.addi" ? " + " : n == "arith.subi" ? " - " : " * ";
      return "(" + cType(rt) + ")((" + u + ")" + arg(0) + o + "(" + u + ")" + arg(1) + ")";
    }
    if (n == "arith.cmpi" || n == "arith.cmpf") return compare(op);
    if (n == "arith.select") return arg(0) + " ? " + arg(1) + " : " + arg(2);
    if (n == "arith.index_cast" || n == "arith.extf" || n == "arith.truncf" || n == "arith.extsi" || n == "arith.trunci" ||
        n == "arith.fptosi" || n == "arith.sitofp")
      return "(" + cType(rt) + ")" + arg(0);
    if (n == "math.exp") return (rt.kind == Type::F32 ? "expf(" : "exp(") + arg(0) + ")";
    if (n == "math.rsqrt") return (rt.kind == Type::F32 ? "rsqrtf(" : "rsqrt(") + arg(0) + ")";
    if (n == "ckl.load_element") return element(op, 0, 1);
    throw CompileError("device code generation does not support '" + n + "'");
  }

  void statement(const Op &op, int indent) {
    const std::string &n = op.name;
    if (n == "func.return") { out << pad(indent) << "return;\n"; return; }
    if (n == "ckl.store_element") {
      out << pad(indent) << element(op, 1, 2) << " = " << ref(op.operands[0]) << ";\n";
      return;
    }
    if (n == "scf.yield") {
      if (yieldTargets.empty()) throw CompileError("scf.yield outside a structured region");
      const auto &targets = yieldTargets.back();
      if (targets.size() != op.operands.size()) throw CompileError("scf.yield arity mismatch");
      std::vector<std::string> temps;
      for (size_t k = 0; k < targets.size(); ++k) {
        std::string t = "y" + std::to_string(next++);
        out << pad(indent) << cType(op.operands[k]->type) << " " << t << " = " << ref(op.operands[k]) << ";\n";
        temps.push_back(t);
      }
      for (size_t k = 0; k < targets.size(); ++k) out << pad(indent) << targets[k] << " = " << temps[k] << ";\n";
      return;
    }
    if (n == "scf.if") {
      std::vector<std::string> targets;
      for (auto &r : op.results) {
        std::string name = bind(r.get());
        out << pad(indent) << cType(r->type) << " " << name << ";\n";
        targets.push_back(name);
      }
      out << pad(indent) << "if (" << ref(op.operands[0]) << ") {\n";
      yieldTargets.push_back(targets);
      region(*op.regions[0], indent + 1);
      out << pad(indent) << "}";
      if (op.regions.size() > 1 && !op.regions[1]->blocks.empty()) {
        out << " else {\n";
        region(*op.regions[1], indent + 1);
        out << pad(indent) << "}";
      }
      out << "\n";
      yieldTargets.pop_back();
      return;
    }
    if (n == "scf.for") {
      const Block &body = *op.regions.at(0)->blocks.at(0);
      std::vector<std::string> carried;
      for (size_t k = 3; k < op.operands.size(); ++k) {
        std::string name = "c" + std::to_string(next++);
        out << pad(indent) << cType(op.operands[k]->type) << " " << name << " = " << ref(op.operands[k]) << ";\n";
        carried.push_back(name);
        names[body.args.at(k - 2).get()] = name;
      }
      std::string iv = bind(body.args.at(0).get());
      out << pad(indent) << "for (long long " << iv << " = " << ref(op.operands[0]) << "; " << iv << " < " << ref(op.operands[1])
          << "; " << iv << " += " << ref(op.operands[2]) << ") {\n";
      yieldTargets.push_back(carried);
      for (auto &child : body.ops) statement(*child, indent + 1);
      yieldTargets.pop_back();
      out << pad(indent) << "}\n";
      for (size_t k = 0; k < op.results.size(); ++k) names[op.results[k].get()] = carried[k];
      return;
    }
    if (op.results.size() != 1) throw CompileError("device code generation does not support '" + n + "'");
    std::string expr = expression(op);
    std::string name = bind(op.results[0].get());
    out << pad(indent) << "const " << cType(op.results[0]->type) << " " << name << " = " << expr << ";\n";
  }

  void region(const Region &r, int indent) {
    for (auto &block : r.blocks)
      for (auto &op : block->ops) statement(*op, indent);
  }
};

std::mutex cacheMutex;
std::map<std::string, std::shared_ptr<const std::vector<uint8_t>>> cache;

void checkRtc(hiprtcResult status, const char *what) {
  if (status != HIPRTC_SUCCESS) throw CompileError(std::string(what) + ": " + hiprtcGetErrorString(status));
}

} // namespace

std::string generateDeviceSource(const Module &prepared, const std::vector<std::string> &kernels) {
  std::ostringstream out;
  out << "// CKL kernels generated for gfx950 (one struct argument per kernel).\n";
  for (const std::string &symbol : kernels) {
    Op *function = prepared.lookup(symbol);
    if (!function || !function->attr("ckl.kernel")) throw CompileError("device code generation: unknown kernel " + symbol);
    KernelEmitter(*function, out).emit();
  }
  return out.str();
}

Artifact compileDeviceCode(const Module &prepared, const std::vector<std::string> &kernels, const std::string &artifact,
                           std::string &source) {
  source = generateDeviceSource(prepared, kernels);
  Artifact result;
  result.identity = artifact;
  result.format = "rocm.hsaco";
  {
    std::lock_guard<std::mutex> lock(cacheMutex);
    auto found = cache.find(artifact);
    if (found != cache.end()) { result.image = found->second; return result; }
  }
  const char *chip = std::getenv("CKL_OFFLOAD_ARCH");
  std::string arch = std::string("--offload-arch=") + (chip ? chip : "gfx950");
  hiprtcProgram program = nullptr;
  checkRtc(hiprtcCreateProgram(&program, source.c_str(), "ckl_generated.hip", 0, nullptr, nullptr), "hiprtcCreateProgram");
  // No floating-point contraction: a*b+c rounds twice, as in the kernel IR.
  const char *options[] = {arch.c_str(), "-O3", "-ffp-contract=off", "-fno-fast-math",
                           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
  hiprtcResult status = hiprtcCompileProgram(program, int(sizeof options / sizeof options[0]), options);
  if (status != HIPRTC_SUCCESS) {
    size_t logSize = 0;
    hiprtcGetProgramLogSize(program, &logSize);
    std::string log(logSize, '\0');
    if (logSize) hiprtcGetProgramLog(program, log.data());
    hiprtcDestroyProgram(&program);
    throw CompileError("hipRTC compilation failed: " + log);
  }
  size_t size = 0;
  checkRtc(hiprtcGetCodeSize(program, &size), "hiprtcGetCodeSize");
  auto image = std::make_shared<std::vector<uint8_t>>(size);
  checkRtc(hiprtcGetCode(program, reinterpret_cast<char *>(image->data())), "hiprtcGetCode");
  hiprtcDestroyProgram(&program);
  {
    std::lock_guard<std::mutex> lock(cacheMutex);
    cache[artifact] = image;
  }
  result.image = image;
  return result;
}

} // namespace ckl::rt
