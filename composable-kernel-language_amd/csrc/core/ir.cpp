// Parser, printer and clone for the CKL IR subset (see ir.h).
#include "ir.h"

#include <algorithm>
#include <cctype>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <sstream>
#include <unordered_map>

namespace ckl {

// ================================================================ types
unsigned Type::bitWidth(Kind k) {
  switch (k) {
  case I1: return 1;
  case I8: return 8;
  case F16: return 16;
  case F32: case I32: return 32;
  case F64: case I64: case Index: return 64;
  default: return 0;
  }
}

std::string kindName(Type::Kind k) {
  switch (k) {
  case Type::None: return "none";
  case Type::F16: return "f16";
  case Type::F32: return "f32";
  case Type::F64: return "f64";
  case Type::I1: return "i1";
  case Type::I8: return "i8";
  case Type::I32: return "i32";
  case Type::I64: return "i64";
  case Type::Index: return "index";
  case Type::Token: return "!ckl.token";
  default: return "?";
  }
}

bool Type::hasStaticShape() const {
  if (kind != MemRef && kind != Vector) return true;
  if (unranked) return false;
  for (int64_t d : shape) if (d < 0) return false;
  return true;
}

int64_t Type::elementCount() const {
  if (!hasStaticShape()) return -1;
  int64_t n = 1;
  for (int64_t d : shape) n *= d;
  return n;
}

std::string Type::str() const {
  switch (kind) {
  case MemRef: case Vector: {
    std::string out = kind == MemRef ? "memref<" : "vector<";
    if (unranked) out += "*x";
    else for (int64_t d : shape) out += (d < 0 ? std::string("?") : std::to_string(d)) + "x";
    out += kindName(element);
    if (!layout.empty()) out += ", " + layout;
    if (!memorySpace.empty()) out += ", " + memorySpace;
    return out + ">";
  }
  case Token: return "!ckl.token";
  case Opaque: return text;
  default: return kindName(kind);
  }
}

// ================================================================ attributes
Attr Attr::dictOf(std::vector<std::pair<std::string, Attr>> entries) {
  std::sort(entries.begin(), entries.end(),
            [](const auto &a, const auto &b) { return a.first < b.first; });
  Attr a; a.kind = Dict; a.dict = std::move(entries); return a;
}

const Attr *Attr::get(const std::string &key) const {
  for (const auto &[k, v] : dict) if (k == key) return &v;
  return nullptr;
}

static std::string quote(const std::string &s) {
  std::string out = "\"";
  for (unsigned char c : s) {
    if (c == '"') out += "\\22";
    else if (c == '\\') out += "\\\\";
    else if (c < 0x20 || c >= 0x7f) { char buf[4]; std::snprintf(buf, sizeof buf, "\\%02X", c); out += buf; }
    else out += char(c);
  }
  return out + "\"";
}

static std::string formatFloat(double v, Type::Kind k) {
  char buf[64];
  if (std::isnan(v) || std::isinf(v)) {
    // Hexadecimal bit pattern, as MLIR prints non-finite values.
    if (k == Type::F32) { float x = float(v); uint32_t bits; std::memcpy(&bits, &x, 4); std::snprintf(buf, sizeof buf, "0x%08X", bits); }
    else { uint64_t bits; std::memcpy(&bits, &v, 8); std::snprintf(buf, sizeof buf, "0x%016llX", (unsigned long long)bits); }
    return buf;
  }
  std::snprintf(buf, sizeof buf, k == Type::F32 ? "%.9e" : "%.17e", v);
  return buf;
}

static bool identifierKey(const std::string &k) {
  if (k.empty() || !(std::isalpha((unsigned char)k[0]) || k[0] == '_')) return false;
  for (char c : k) if (!(std::isalnum((unsigned char)c) || c == '_' || c == '.' || c == '$')) return false;
  return true;
}

static std::string printDict(const std::vector<std::pair<std::string, Attr>> &entries) {
  std::string out = "{";
  bool first = true;
  for (const auto &[k, v] : entries) {
    if (!first) out += ", ";
    first = false;
    out += identifierKey(k) ? k : quote(k);
    if (v.kind != Attr::Unit) out += " = " + v.str();
  }
  return out + "}";
}

std::string Attr::str() const {
  switch (kind) {
  case Null: return "<<null>>";
  case Int:
    if (type.kind == Type::I1) return i ? "true" : "false";
    return std::to_string(i) + " : " + type.str();
  case Float: return formatFloat(f, type.kind) + " : " + type.str();
  case String: return quote(s);
  case Bool: return i ? "true" : "false";
  case Unit: return "unit";
  case Array: {
    // As in MLIR's printer, an i64 integer directly inside an array is printed without its type.
    std::string out = "[";
    for (size_t k = 0; k < array.size(); ++k) {
      const Attr &e = array[k];
      out += (k ? ", " : "") + (e.kind == Int && e.type.kind == Type::I64 ? std::to_string(e.i) : e.str());
    }
    return out + "]";
  }
  case DenseI64: case DenseI32: case DenseI8: {
    std::string out = kind == DenseI64 ? "array<i64" : kind == DenseI32 ? "array<i32" : "array<i8";
    for (size_t k = 0; k < dense.size(); ++k) out += (k ? ", " : ": ") + std::to_string(dense[k]);
    return out + ">";
  }
  case Symbol: {
    std::string out = "@" + s;
    for (const auto &n : nested) out += "::@" + n;
    return out;
  }
  case Dict: return printDict(dict);
  case TypeAttr: return type.str();
  }
  return "?";
}

// ================================================================ ops
Op *Op::parentOp() const {
  return parent && parent->parent ? parent->parent->parent : nullptr;
}

std::string Op::symName() const {
  const Attr *a = attr("sym_name");
  return a ? a->s : std::string();
}

Block *Op::entry() const {
  if (regions.empty() || regions[0]->blocks.empty()) return nullptr;
  return regions[0]->blocks[0].get();
}

std::vector<Op *> Module::functions() const {
  std::vector<Op *> out;
  for (auto &op : body()->ops) if (op->name == "func.func") out.push_back(op.get());
  return out;
}

Op *Module::lookup(const std::string &symbol) const {
  for (auto &op : body()->ops) if (op->symName() == symbol) return op.get();
  return nullptr;
}

std::string sourcePosition(const Op *op) {
  if (!op->loc.empty()) return op->loc + ": ";
  if (op->line) return std::to_string(op->line) + ":" + std::to_string(op->column) + ": ";
  return {};
}

void walkPreOrder(Op *op, const std::function<void(Op *)> &fn) {
  fn(op);
  for (auto &region : op->regions)
    for (auto &block : region->blocks)
      for (auto &child : block->ops) walkPreOrder(child.get(), fn);
}

// ================================================================ parser
namespace {

class Parser {
public:
  explicit Parser(const std::string &text) : s(text) {
    lineStarts.push_back(0);
    for (size_t k = 0; k < s.size(); ++k)
      if (s[k] == '\n') lineStarts.push_back(k + 1);
  }

  std::unique_ptr<Module> parse() {
    auto module = std::make_unique<Module>();
    module->op = std::make_unique<Op>();
    module->op->name = "builtin.module";
    auto region = std::make_unique<Region>();
    region->parent = module->op.get();
    auto block = std::make_unique<Block>();
    block->parent = region.get();
    Block *body = block.get();
    region->blocks.push_back(std::move(block));
    module->op->regions.push_back(std::move(region));
    ws();
    if (keyword("module")) {
      ws();
      if (keyword("attributes")) { ws(); parseAttrDictInto(module->op->attrs); ws(); }
      expect("{");
      pushScope();
      parseOpsUntil(body, "}");
      popScope();
      expect("}");
    } else {
      pushScope();
      parseOpsUntil(body, "");
      popScope();
    }
    ws();
    if (pos < s.size()) fail("unexpected trailing text");
    return module;
  }

private:
  const std::string &s;
  size_t pos = 0;
  std::vector<std::unordered_map<std::string, Value *>> scopes;

  std::vector<size_t> lineStarts;   // offset of the first character of each line

  // 1-based line and column of a text offset.
  std::pair<unsigned, unsigned> position(size_t offset) const {
    offset = std::min(offset, s.size());
    size_t line = size_t(std::upper_bound(lineStarts.begin(), lineStarts.end(), offset) - lineStarts.begin());
    return {unsigned(line), unsigned(offset - lineStarts[line - 1] + 1)};
  }

  [[noreturn]] void fail(const std::string &message) const {
    auto [line, column] = position(pos);
    throw IRError(std::to_string(line) + ":" + std::to_string(column) + ": " + message);
  }

  void ws() {
    while (pos < s.size()) {
      if (std::isspace((unsigned char)s[pos])) ++pos;
      else if (s.compare(pos, 2, "//") == 0) { while (pos < s.size() && s[pos] != '\n') ++pos; }
      else break;
    }
  }
  bool peek(const char *t) { ws(); return s.compare(pos, std::strlen(t), t) == 0; }
  bool consume(const char *t) { if (peek(t)) { pos += std::strlen(t); return true; } return false; }
  void expect(const char *t) { if (!consume(t)) fail(std::string("expected '") + t + "'"); }
  static bool identChar(char c) { return std::isalnum((unsigned char)c) || c == '_' || c == '.' || c == '$' || c == '-'; }
  bool keyword(const char *k) {
    ws();
    size_t n = std::strlen(k);
    if (s.compare(pos, n, k) == 0 && (pos + n >= s.size() || !identChar(s[pos + n]))) { pos += n; return true; }
    return false;
  }
  std::string bareIdent() {
    ws();
    size_t start = pos;
    if (pos < s.size() && (std::isalpha((unsigned char)s[pos]) || s[pos] == '_')) {
      ++pos;
      while (pos < s.size() && (std::isalnum((unsigned char)s[pos]) || s[pos] == '_' || s[pos] == '.' || s[pos] == '$')) ++pos;
    }
    if (start == pos) fail("expected identifier");
    return s.substr(start, pos - start);
  }
  std::string stringLiteral() {
    ws();
    if (pos >= s.size() || s[pos] != '"') fail("expected string literal");
    ++pos;
    std::string out;
    while (pos < s.size() && s[pos] != '"') {
      char c = s[pos++];
      if (c == '\\') {
        if (pos >= s.size()) fail("unterminated escape");
        char n = s[pos];
        if (n == '\\' || n == '"') { out += n; ++pos; }
        else if (n == 'n') { out += '\n'; ++pos; }
        else if (n == 't') { out += '\t'; ++pos; }
        else if (std::isxdigit((unsigned char)n) && pos + 1 < s.size() && std::isxdigit((unsigned char)s[pos + 1])) {
          out += char(std::stoi(s.substr(pos, 2), nullptr, 16)); pos += 2;
        } else fail("invalid escape in string literal");
      } else out += c;
    }
    if (pos >= s.size()) fail("unterminated string literal");
    ++pos;
    return out;
  }
  std::string valueName() {
    ws();
    if (pos >= s.size() || s[pos] != '%') fail("expected SSA value");
    size_t start = ++pos;
    while (pos < s.size() && (std::isalnum((unsigned char)s[pos]) || s[pos] == '_' || s[pos] == '.' || s[pos] == '$' || s[pos] == '-' || s[pos] == '#')) ++pos;
    if (start == pos) fail("empty SSA value name");
    return s.substr(start, pos - start);
  }
  std::string symbolName() {
    ws();
    if (!consume("@")) fail("expected symbol");
    if (pos < s.size() && s[pos] == '"') return stringLiteral();
    return bareIdent();
  }

  void pushScope() { scopes.emplace_back(); }
  void popScope() { scopes.pop_back(); }
  void define(const std::string &name, Value *v) {
    auto &scope = scopes.back();
    if (scope.count(name)) fail("redefinition of SSA value %" + name);
    scope[name] = v;
  }
  Value *lookup(const std::string &name) {
    // '#' result selectors: %x#1
    std::string base = name;
    unsigned index = 0;
    auto hash = name.find('#');
    if (hash != std::string::npos) { base = name.substr(0, hash); index = std::stoul(name.substr(hash + 1)); }
    for (auto it = scopes.rbegin(); it != scopes.rend(); ++it) {
      auto found = it->find(base);
      if (found != it->end()) {
        Value *v = found->second;
        if (index) {
          if (!v->def || index >= v->def->results.size()) fail("invalid result selector %" + name);
          return v->def->results[index].get();
        }
        return v;
      }
    }
    fail("use of undefined SSA value %" + name);
  }
  Value *operand() { return lookup(valueName()); }

  // ------------------------------------------------------------ types
  Type::Kind scalarKind(const std::string &t) {
    static const std::map<std::string, Type::Kind> kinds = {
        {"f16", Type::F16}, {"f32", Type::F32}, {"f64", Type::F64}, {"i1", Type::I1}, {"i8", Type::I8},
        {"i32", Type::I32}, {"i64", Type::I64}, {"index", Type::Index}, {"none", Type::None}};
    auto it = kinds.find(t);
    return it == kinds.end() ? Type::Opaque : it->second;
  }
  std::string balanced(char open, char close) {
    size_t start = pos;
    int depth = 0;
    while (pos < s.size()) {
      char c = s[pos];
      if (c == '"') { stringLiteral(); continue; }
      if (c == open) ++depth;
      else if (c == close) { if (--depth == 0) { ++pos; return s.substr(start, pos - start); } }
      ++pos;
    }
    fail("unbalanced brackets");
  }
  Type parseType() {
    ws();
    Type t;
    if (consume("!ckl.token")) { t.kind = Type::Token; return t; }
    if (peek("!")) {
      size_t start = pos++;
      while (pos < s.size() && (std::isalnum((unsigned char)s[pos]) || s[pos] == '_' || s[pos] == '.')) ++pos;
      if (pos < s.size() && s[pos] == '<') balanced('<', '>');
      t.kind = Type::Opaque; t.text = s.substr(start, pos - start);
      return t;
    }
    bool mem = keyword("memref");
    bool vec = !mem && keyword("vector");
    if (mem || vec) {
      t.kind = mem ? Type::MemRef : Type::Vector;
      expect("<");
      if (consume("*")) { t.unranked = true; expect("x"); }
      else {
        while (true) {
          ws();
          if (pos < s.size() && s[pos] == '?') { ++pos; t.shape.push_back(-1); expect("x"); continue; }
          if (pos < s.size() && std::isdigit((unsigned char)s[pos])) {
            size_t start = pos;
            while (pos < s.size() && std::isdigit((unsigned char)s[pos])) ++pos;
            t.shape.push_back(std::stoll(s.substr(start, pos - start)));
            if (pos < s.size() && s[pos] == 'x') { ++pos; continue; }
            fail("expected 'x' in shaped type");
          }
          break;
        }
      }
      std::string elem = bareIdent();
      t.element = scalarKind(elem);
      if (t.element == Type::Opaque || t.element == Type::None) fail("unsupported element type " + elem);
      // Optional layout, then optional memory space: memref<4xf32, strided<[1], offset: 4>, 3>.
      while (consume(",")) {
        ws();
        size_t start = pos;
        int depth = 0;
        while (pos < s.size() && !(depth == 0 && (s[pos] == '>' || s[pos] == ','))) {
          if (s[pos] == '<' || s[pos] == '(' || s[pos] == '[') ++depth;
          if (s[pos] == '>' || s[pos] == ')' || s[pos] == ']') --depth;
          ++pos;
        }
        std::string extra = s.substr(start, pos - start);
        while (!extra.empty() && std::isspace((unsigned char)extra.back())) extra.pop_back();
        if (extra.empty()) fail("expected memref layout or memory space");
        if (extra.rfind("strided", 0) == 0 || extra.rfind("affine_map", 0) == 0) {
          if (!t.layout.empty() || !t.memorySpace.empty()) fail("memref layout must precede the memory space");
          t.identityLayout = false;
          t.layout = extra;
        } else {
          if (!t.memorySpace.empty()) fail("duplicate memref memory space");
          t.memorySpace = extra;
        }
      }
      expect(">");
      return t;
    }
    std::string name = bareIdent();
    Type::Kind k = scalarKind(name);
    if (k == Type::Opaque) { t.kind = Type::Opaque; t.text = name; return t; }
    t.kind = k;
    return t;
  }
  std::vector<Type> typeList() {
    std::vector<Type> out;
    expect("(");
    if (consume(")")) return out;
    do out.push_back(parseType()); while (consume(","));
    expect(")");
    return out;
  }
  void functionType(std::vector<Type> &inputs, std::vector<Type> &outputs) {
    inputs = typeList();
    expect("->");
    if (peek("(")) outputs = typeList();
    else outputs.push_back(parseType());
  }

  // ------------------------------------------------------------ attributes
  Attr parseAttr() {
    ws();
    if (pos >= s.size()) fail("expected attribute");
    char c = s[pos];
    if (c == '"') return Attr::string(stringLiteral());
    if (c == '[') {
      ++pos;
      Attr a; a.kind = Attr::Array;
      if (!consume("]")) { do a.array.push_back(parseAttr()); while (consume(",")); expect("]"); }
      return a;
    }
    if (c == '{') {
      std::map<std::string, Attr> entries;
      parseAttrDictInto(entries);
      return Attr::dictOf({entries.begin(), entries.end()});
    }
    if (c == '@') {
      Attr a = Attr::symbol(symbolName());
      while (consume("::")) a.nested.push_back(symbolName());
      return a;
    }
    if (keyword("true")) return Attr::boolean(true);
    if (keyword("false")) return Attr::boolean(false);
    if (keyword("unit")) return Attr::unit();
    if (peek("array<")) {
      pos += 6;
      std::string elem = bareIdent();
      Attr a;
      a.kind = elem == "i64" ? Attr::DenseI64 : elem == "i32" ? Attr::DenseI32 : elem == "i8" ? Attr::DenseI8 : Attr::Null;
      if (a.kind == Attr::Null) fail("unsupported dense array element " + elem);
      if (consume(":")) { do a.dense.push_back(parseInteger()); while (consume(",")); }
      expect(">");
      return a;
    }
    if (c == '-' || c == '+' || std::isdigit((unsigned char)c)) {
      size_t start = pos;
      bool hex = s.compare(pos, 2, "0x") == 0 || s.compare(pos, 2, "0X") == 0;
      if (c == '-' || c == '+') ++pos;
      bool isFloat = false;
      if (hex) { pos += 2; while (pos < s.size() && std::isxdigit((unsigned char)s[pos])) ++pos; }
      else {
        while (pos < s.size() && (std::isdigit((unsigned char)s[pos]) || s[pos] == '.' || s[pos] == 'e' || s[pos] == 'E' ||
                                  ((s[pos] == '-' || s[pos] == '+') && (s[pos - 1] == 'e' || s[pos - 1] == 'E')))) {
          if (s[pos] == '.' || s[pos] == 'e' || s[pos] == 'E') isFloat = true;
          ++pos;
        }
      }
      std::string literal = s.substr(start, pos - start);
      Type t = Type::scalar(isFloat ? Type::F64 : Type::I64);
      if (consume(":")) t = parseType();
      if (t.isFloat()) {
        double v;
        if (hex) {
          unsigned long long bits = std::stoull(literal, nullptr, 16);
          if (t.kind == Type::F32) { uint32_t b32 = uint32_t(bits); float x; std::memcpy(&x, &b32, 4); v = x; }
          else std::memcpy(&v, &bits, 8);
        } else v = std::stod(literal);
        if (t.kind == Type::F32) v = double(float(v));
        return Attr::floating(v, t.kind);
      }
      if (isFloat) fail("float literal requires a float type");
      Attr a = Attr::integer(hex ? (int64_t)std::stoull(literal, nullptr, 16) : std::stoll(literal), Type::I64);
      a.type = t;
      return a;
    }
    // Bare type attributes (e.g. type = f32 / memref<4xf32>)
    Attr a; a.kind = Attr::TypeAttr; a.type = parseType();
    return a;
  }
  int64_t parseInteger() {
    ws();
    size_t start = pos;
    if (pos < s.size() && (s[pos] == '-' || s[pos] == '+')) ++pos;
    while (pos < s.size() && std::isdigit((unsigned char)s[pos])) ++pos;
    if (start == pos) fail("expected integer");
    return std::stoll(s.substr(start, pos - start));
  }
  void parseAttrDictInto(std::map<std::string, Attr> &into) {
    expect("{");
    if (consume("}")) return;
    do {
      ws();
      std::string key = (pos < s.size() && s[pos] == '"') ? stringLiteral() : bareIdent();
      if (consume("=")) into[key] = parseAttr();
      else into[key] = Attr::unit();
    } while (consume(","));
    expect("}");
  }
  std::string location() {
    // loc(...) with balanced parentheses; returns the inner text.
    if (!peek("loc(")) return {};
    pos += 3;
    std::string text = balanced('(', ')');
    return text.substr(1, text.size() - 2);
  }

  // ------------------------------------------------------------ ops
  Op *append(Block *block, std::unique_ptr<Op> op) {
    op->parent = block;
    Op *raw = op.get();
    block->ops.push_back(std::move(op));
    return raw;
  }
  void addResults(Op *op, const std::vector<Type> &types, const std::vector<std::string> &names) {
    for (size_t k = 0; k < types.size(); ++k) {
      auto v = std::make_unique<Value>();
      v->type = types[k]; v->def = op; v->index = unsigned(k);
      op->results.push_back(std::move(v));
    }
    bindResults(op, names);
  }
  void bindResults(Op *op, const std::vector<std::string> &names) {
    if (names.empty()) return;
    if (names.size() == 1 && op->results.size() >= 1) {
      op->results[0]->hint = names[0];
      define(names[0], op->results[0].get());
      return;
    }
    if (names.size() != op->results.size()) fail("result count mismatch");
    for (size_t k = 0; k < names.size(); ++k) { op->results[k]->hint = names[k]; define(names[k], op->results[k].get()); }
  }

  void parseOpsUntil(Block *block, const char *terminator) {
    while (true) {
      ws();
      if (pos >= s.size()) { if (*terminator) fail(std::string("expected '") + terminator + "'"); return; }
      if (*terminator && peek(terminator)) return;
      if (peek("^")) return;  // next block label
      parseOperation(block);
    }
  }

  std::unique_ptr<Region> parseRegion(Op *owner, const std::vector<std::pair<std::string, Type>> &entryArgs = {}) {
    auto region = std::make_unique<Region>();
    region->parent = owner;
    expect("{");
    pushScope();
    bool first = true;
    while (true) {
      ws();
      if (consume("}")) break;
      auto block = std::make_unique<Block>();
      block->parent = region.get();
      if (peek("^")) {
        ++pos;
        bareIdent();
        if (consume("(")) {
          if (!consume(")")) {
            do {
              std::string name = valueName();
              expect(":");
              Type t = parseType();
              auto v = std::make_unique<Value>();
              v->type = t; v->owner = block.get(); v->index = unsigned(block->args.size()); v->hint = name;
              define(name, v.get());
              block->args.push_back(std::move(v));
            } while (consume(","));
            expect(")");
          }
        }
        expect(":");
      } else if (first) {
        for (auto &[name, t] : entryArgs) {
          auto v = std::make_unique<Value>();
          v->type = t; v->owner = block.get(); v->index = unsigned(block->args.size()); v->hint = name;
          if (!name.empty()) define(name, v.get());
          block->args.push_back(std::move(v));
        }
      }
      first = false;
      Block *raw = block.get();
      region->blocks.push_back(std::move(block));
      parseOpsUntil(raw, "}");
    }
    popScope();
    return region;
  }

  void parseOperation(Block *block) {
    std::vector<std::string> names;
    ws();
    auto [line, column] = position(pos);
    parseOperationAt(block, names);
    Op *op = block->ops.back().get();
    op->line = line;
    op->column = column;
  }

  void parseOperationAt(Block *block, std::vector<std::string> &names) {
    if (peek("%")) {
      do {
        std::string name = valueName();
        if (consume(":")) {   // %x:2 = ... result packs
          int64_t count = parseInteger();
          for (int64_t k = 0; k < count; ++k) names.push_back(k ? name + "#" + std::to_string(k) : name);
          continue;
        }
        names.push_back(name);
      } while (consume(","));
      expect("=");
    }
    ws();
    if (pos < s.size() && s[pos] == '"') { parseGeneric(block, names); return; }
    std::string name = bareIdent();
    parsePretty(block, name, names);
  }

  void parseGeneric(Block *block, const std::vector<std::string> &names) {
    auto op = std::make_unique<Op>();
    op->name = stringLiteral();
    Op *raw = op.get();
    append(block, std::move(op));
    expect("(");
    if (!consume(")")) { do raw->operands.push_back(operand()); while (consume(",")); expect(")"); }
    if (consume("<")) { parseAttrDictInto(raw->attrs); expect(">"); }
    if (consume("(")) {
      do raw->regions.push_back(parseRegion(raw)); while (consume(","));
      expect(")");
    }
    if (peek("{")) parseAttrDictInto(raw->attrs);
    expect(":");
    std::vector<Type> inputs, outputs;
    functionType(inputs, outputs);
    if (inputs.size() != raw->operands.size()) fail("operand type count does not match operands of " + raw->name);
    for (size_t k = 0; k < inputs.size(); ++k)
      if (inputs[k] != raw->operands[k]->type) fail("operand type mismatch for " + raw->name);
    addResults(raw, outputs, names);
    raw->loc = location();
  }

  std::unique_ptr<Op> make(const std::string &name) { auto op = std::make_unique<Op>(); op->name = name; return op; }

  void parseFunc(Block *block, const std::string &opName) {
    auto op = make(opName);
    Op *raw = append(block, std::move(op));
    if (keyword("private")) raw->attrs["sym_visibility"] = Attr::string("private");
    else if (keyword("public")) {}
    std::string symbol = symbolName();
    raw->attrs["sym_name"] = Attr::string(symbol);
    std::vector<std::pair<std::string, Type>> args;
    std::vector<Type> inputs, outputs;
    expect("(");
    if (!consume(")")) {
      do {
        ws();
        if (peek("%")) {
          std::string name = valueName();
          expect(":");
          Type t = parseType();
          if (peek("{")) { std::map<std::string, Attr> ignored; parseAttrDictInto(ignored); }
          args.emplace_back(name, t);
          inputs.push_back(t);
        } else {
          inputs.push_back(parseType());
          args.emplace_back("", inputs.back());
        }
      } while (consume(","));
      expect(")");
    }
    if (consume("->")) {
      if (peek("(")) outputs = typeList();
      else outputs.push_back(parseType());
    }
    if (keyword("attributes")) parseAttrDictInto(raw->attrs);
    Attr ft; ft.kind = Attr::TypeAttr; ft.type.kind = Type::Opaque;
    std::string sig = "(";
    for (size_t k = 0; k < inputs.size(); ++k) sig += (k ? ", " : "") + inputs[k].str();
    sig += ") -> ";
    if (outputs.size() == 1) sig += outputs[0].str();
    else { sig += "("; for (size_t k = 0; k < outputs.size(); ++k) sig += (k ? ", " : "") + outputs[k].str(); sig += ")"; }
    ft.type.text = sig;
    raw->attrs["function_type"] = ft;
    raw->attrs["ckl.num_results"] = Attr::integer(int64_t(outputs.size()));
    if (peek("{")) {
      for (auto &arg : args) if (arg.first.empty()) fail("function definition requires named arguments");
      raw->regions.push_back(parseRegion(raw, args));
    } else {
      // Declarations keep their argument types in an empty region-less op.
      std::vector<Attr> types;
      for (auto &t : inputs) types.push_back(Attr::typeAttr(t));
      raw->attrs["ckl.argument_types"] = Attr::arrayOf(types);
    }
    raw->loc = location();
  }

  void parsePretty(Block *block, const std::string &name, const std::vector<std::string> &names) {
    if (name == "func.func" || name == "func") { parseFunc(block, "func.func"); return; }
    auto op = make(name == "return" ? "func.return" : name);
    Op *raw = append(block, std::move(op));
    const std::string &n = raw->name;
    std::vector<Type> results;
    auto binaryOps = [](const std::string &x) {
      static const char *names[] = {"arith.addf", "arith.subf", "arith.mulf", "arith.divf", "arith.addi",
                                    "arith.subi", "arith.muli", "arith.divsi", "arith.remsi", "arith.maximumf",
                                    "arith.minimumf", "arith.andi", "arith.ori", "arith.xori"};
      for (const char *c : names) if (x == c) return true;
      return false;
    };
    if (n == "func.return" || n == "scf.yield") {
      ws();
      if (peek("%")) {
        do raw->operands.push_back(operand()); while (consume(","));
        expect(":");
        do parseType(); while (consume(","));
      }
    } else if (n == "arith.constant") {
      Attr value = parseAttr();
      if (value.kind == Attr::Bool) { value = Attr::integer(value.i, Type::I1); }
      raw->attrs["value"] = value;
      results.push_back(value.type);
    } else if (binaryOps(n)) {
      raw->operands.push_back(operand()); expect(","); raw->operands.push_back(operand());
      expect(":"); results.push_back(parseType());
    } else if (n == "arith.negf" || n == "math.exp" || n == "math.rsqrt" || n == "math.sqrt") {
      raw->operands.push_back(operand()); expect(":"); results.push_back(parseType());
    } else if (n == "arith.cmpi" || n == "arith.cmpf") {
      std::string predicate = bareIdent();
      static const std::map<std::string, int> ipred = {{"eq", 0}, {"ne", 1}, {"slt", 2}, {"sle", 3}, {"sgt", 4}, {"sge", 5}, {"ult", 6}, {"ule", 7}, {"ugt", 8}, {"uge", 9}};
      static const std::map<std::string, int> fpred = {{"false", 0}, {"oeq", 1}, {"ogt", 2}, {"oge", 3}, {"olt", 4}, {"ole", 5}, {"one", 6}, {"ord", 7}, {"ueq", 8}, {"ugt", 9}, {"uge", 10}, {"ult", 11}, {"ule", 12}, {"une", 13}, {"uno", 14}, {"true", 15}};
      const auto &table = n == "arith.cmpi" ? ipred : fpred;
      auto it = table.find(predicate);
      if (it == table.end()) fail("unknown comparison predicate " + predicate);
      raw->attrs["predicate"] = Attr::integer(it->second);
      expect(",");
      raw->operands.push_back(operand()); expect(","); raw->operands.push_back(operand());
      expect(":"); parseType();
      results.push_back(Type::scalar(Type::I1));
    } else if (n == "arith.select") {
      raw->operands.push_back(operand()); expect(",");
      raw->operands.push_back(operand()); expect(",");
      raw->operands.push_back(operand());
      expect(":"); results.push_back(parseType());
    } else if (n == "arith.index_cast" || n == "arith.extf" || n == "arith.truncf" || n == "arith.extsi" ||
               n == "arith.trunci" || n == "arith.fptosi" || n == "arith.sitofp" || n == "arith.bitcast") {
      raw->operands.push_back(operand()); expect(":"); parseType();
      if (!keyword("to")) fail("expected 'to'");
      results.push_back(parseType());
    } else if (n == "scf.if") {
      raw->operands.push_back(operand());
      if (consume("->")) results = typeList();
      raw->regions.push_back(parseRegion(raw));
      if (keyword("else")) raw->regions.push_back(parseRegion(raw));
      else { auto empty = std::make_unique<Region>(); empty->parent = raw; raw->regions.push_back(std::move(empty)); }
    } else if (n == "scf.for") {
      std::string iv = valueName();
      expect("=");
      raw->operands.push_back(operand());
      if (!keyword("to")) fail("expected 'to'");
      raw->operands.push_back(operand());
      if (!keyword("step")) fail("expected 'step'");
      raw->operands.push_back(operand());
      std::vector<std::pair<std::string, Type>> args = {{iv, Type::scalar(Type::Index)}};
      if (keyword("iter_args")) {
        expect("(");
        std::vector<std::string> carried;
        do { carried.push_back(valueName()); expect("="); raw->operands.push_back(operand()); } while (consume(","));
        expect(")");
        expect("->");
        results = typeList();
        if (results.size() != carried.size()) fail("iter_args/result count mismatch");
        for (size_t k = 0; k < carried.size(); ++k) args.emplace_back(carried[k], results[k]);
      }
      raw->regions.push_back(parseRegion(raw, args));
    } else if (n == "memref.alloc") {
      expect("(");
      if (!consume(")")) { do raw->operands.push_back(operand()); while (consume(",")); expect(")"); }
      expect(":");
      results.push_back(parseType());
    } else if (n == "memref.dealloc") {
      raw->operands.push_back(operand()); expect(":"); parseType();
    } else if (n == "memref.load") {
      raw->operands.push_back(operand());
      expect("[");
      if (!consume("]")) { do raw->operands.push_back(operand()); while (consume(",")); expect("]"); }
      expect(":");
      Type m = parseType();
      results.push_back(Type::scalar(m.element));
    } else if (n == "memref.store") {
      raw->operands.push_back(operand()); expect(",");
      raw->operands.push_back(operand());
      expect("[");
      if (!consume("]")) { do raw->operands.push_back(operand()); while (consume(",")); expect("]"); }
      expect(":"); parseType();
    } else if (n == "memref.copy") {
      raw->operands.push_back(operand()); expect(",");
      raw->operands.push_back(operand());
      expect(":");
      if (parseType() != raw->operands[0]->type) fail("memref.copy source type does not match its operand");
      if (!keyword("to")) fail("expected 'to'");
      if (parseType() != raw->operands[1]->type) fail("memref.copy target type does not match its operand");
    } else if (n == "memref.subview") {
      // Static offsets, sizes and strides only; kept in the attributes of MLIR's generic form.
      raw->operands.push_back(operand());
      auto staticList = [&](const char *key) {
        expect("[");
        std::vector<int64_t> values;
        if (!consume("]")) {
          do {
            if (peek("%")) fail("memref.subview with dynamic offsets, sizes or strides is unsupported");
            values.push_back(parseInteger());
          } while (consume(","));
          expect("]");
        }
        raw->attrs[key] = Attr::denseI64(values);
      };
      staticList("static_offsets");
      staticList("static_sizes");
      staticList("static_strides");
      raw->attrs["operandSegmentSizes"] = Attr::denseI32({1, 0, 0, 0});
      expect(":");
      if (parseType() != raw->operands[0]->type) fail("memref.subview source type does not match its operand");
      if (!keyword("to")) fail("expected 'to'");
      results.push_back(parseType());
    } else if (n == "func.call") {
      raw->attrs["callee"] = Attr::symbol(symbolName());
      expect("(");
      if (!consume(")")) { do raw->operands.push_back(operand()); while (consume(",")); expect(")"); }
      expect(":");
      std::vector<Type> inputs;
      functionType(inputs, results);
      if (results.size() == 1 && results[0].kind == Type::None) results.clear();
    } else {
      fail("unsupported custom operation syntax '" + n + "'");
    }
    if (peek("{") && n != "scf.if" && n != "scf.for") parseAttrDictInto(raw->attrs);
    addResults(raw, results, names);
    raw->loc = location();
  }
};

} // namespace

std::unique_ptr<Module> parseModule(const std::string &text) { return Parser(text).parse(); }

// ================================================================ printer
namespace {

class Printer {
public:
  explicit Printer(bool locations) : locations(locations) {}
  std::string out;

  void module(const Module &m) {
    out += "module";
    if (!m.op->attrs.empty()) {
      out += " attributes ";
      out += printDict({m.op->attrs.begin(), m.op->attrs.end()});
    }
    out += " {\n";
    for (auto &op : m.body()->ops) operation(*op, 1);
    out += "}\n";
  }

  void operation(const Op &op, int indent) {
    std::string pad(indent * 2, ' ');
    if (op.name == "func.func") { function(op, indent); return; }
    out += pad;
    if (!op.results.empty()) {
      for (size_t k = 0; k < op.results.size(); ++k) out += (k ? ", " : "") + name(op.results[k].get());
      out += " = ";
    }
    out += quote(op.name) + "(";
    for (size_t k = 0; k < op.operands.size(); ++k) out += (k ? ", " : "") + name(op.operands[k]);
    out += ")";
    if (!op.regions.empty()) {
      out += " (";
      for (size_t r = 0; r < op.regions.size(); ++r) {
        out += r ? ", {\n" : "{\n";
        region(*op.regions[r], indent + 1);
        out += pad + "}";
      }
      out += ")";
    }
    std::vector<std::pair<std::string, Attr>> attrs;
    for (auto &[k, v] : op.attrs) if (k.rfind("ckl.internal.", 0) != 0) attrs.emplace_back(k, v);
    if (!attrs.empty()) out += " " + printDict(attrs);
    out += " : (";
    for (size_t k = 0; k < op.operands.size(); ++k) out += (k ? ", " : "") + op.operands[k]->type.str();
    out += ") -> ";
    if (op.results.size() == 1) out += op.results[0]->type.str();
    else {
      out += "(";
      for (size_t k = 0; k < op.results.size(); ++k) out += (k ? ", " : "") + op.results[k]->type.str();
      out += ")";
    }
    if (locations && !op.loc.empty()) out += " loc(" + op.loc + ")";
    out += "\n";
  }

  void region(const Region &r, int indent) {
    for (size_t b = 0; b < r.blocks.size(); ++b) {
      const Block &block = *r.blocks[b];
      if (!block.args.empty()) {
        out += std::string(indent * 2 - 2, ' ') + "^bb" + std::to_string(b) + "(";
        for (size_t k = 0; k < block.args.size(); ++k)
          out += (k ? ", " : "") + name(block.args[k].get()) + ": " + block.args[k]->type.str();
        out += "):\n";
      }
      for (auto &op : block.ops) operation(*op, indent);
    }
  }

  void function(const Op &op, int indent) {
    std::string pad(indent * 2, ' ');
    out += pad + "func.func ";
    if (const Attr *v = op.attr("sym_visibility")) out += v->s + " ";
    out += "@" + op.symName() + "(";
    Block *entry = op.entry();
    if (entry) {
      for (size_t k = 0; k < entry->args.size(); ++k)
        out += (k ? ", " : "") + name(entry->args[k].get()) + ": " + entry->args[k]->type.str();
    } else if (const Attr *types = op.attr("ckl.argument_types")) {
      for (size_t k = 0; k < types->array.size(); ++k) out += (k ? ", " : "") + types->array[k].type.str();
    }
    out += ")";
    std::vector<std::pair<std::string, Attr>> attrs;
    for (auto &[k, v] : op.attrs)
      if (k != "sym_name" && k != "function_type" && k != "sym_visibility" && k != "ckl.num_results" &&
          k != "ckl.argument_types" && k.rfind("ckl.internal.", 0) != 0)
        attrs.emplace_back(k, v);
    if (!attrs.empty()) out += " attributes " + printDict(attrs);
    if (entry) {
      out += " {\n";
      for (size_t b = 0; b < op.regions[0]->blocks.size(); ++b) {
        const Block &block = *op.regions[0]->blocks[b];
        if (b) {
          out += pad + "^bb" + std::to_string(b) + "(";
          for (size_t k = 0; k < block.args.size(); ++k)
            out += (k ? ", " : "") + name(block.args[k].get()) + ": " + block.args[k]->type.str();
          out += "):\n";
        }
        for (auto &child : block.ops) operation(*child, indent + 1);
      }
      out += pad + "}";
    }
    if (locations && !op.loc.empty()) out += " loc(" + op.loc + ")";
    out += "\n";
  }

private:
  bool locations;
  std::unordered_map<const Value *, std::string> names;
  unsigned nextValue = 0, nextArg = 0;

  std::string name(const Value *v) {
    auto it = names.find(v);
    if (it != names.end()) return it->second;
    std::string n = v->def ? "%" + std::to_string(nextValue++) : "%arg" + std::to_string(nextArg++);
    names[v] = n;
    return n;
  }
};

} // namespace

std::string printModule(const Module &module, bool locations) {
  Printer p(locations);
  p.module(module);
  return p.out;
}

std::string printOp(const Op &op, bool locations, int indent) {
  Printer p(locations);
  p.operation(op, indent);
  return p.out;
}

std::string canonicalFunction(const Op &function) {
  Printer p(false);
  Op copy;
  (void)copy;
  p.function(function, 0);
  // Drop the symbol name: "func.func [vis] @name(" -> "func.func (".
  std::string text = p.out;
  size_t at = text.find('@');
  size_t paren = text.find('(', at);
  if (at != std::string::npos && paren != std::string::npos) text.erase(at, paren - at);
  return text;
}

// ================================================================ clone
namespace {
struct Cloner {
  ValueMap own;
  ValueMap &map = own;

  std::unique_ptr<Op> op(const Op &src, Block *parent) {
    auto out = std::make_unique<Op>();
    out->name = src.name;
    out->attrs = src.attrs;
    out->loc = src.loc;
    out->parent = parent;
    for (Value *v : src.operands) {
      auto it = map.find(v);
      out->operands.push_back(it == map.end() ? v : it->second);
    }
    for (auto &r : src.results) {
      auto v = std::make_unique<Value>(*r);
      v->def = out.get();
      map[r.get()] = v.get();
      out->results.push_back(std::move(v));
    }
    for (auto &region : src.regions) out->regions.push_back(this->region(*region, out.get()));
    return out;
  }

  std::unique_ptr<Region> region(const Region &src, Op *owner) {
    auto out = std::make_unique<Region>();
    out->parent = owner;
    for (auto &block : src.blocks) {
      auto b = std::make_unique<Block>();
      b->parent = out.get();
      for (auto &arg : block->args) {
        auto v = std::make_unique<Value>(*arg);
        v->owner = b.get();
        map[arg.get()] = v.get();
        b->args.push_back(std::move(v));
      }
      out->blocks.push_back(std::move(b));
    }
    for (size_t k = 0; k < src.blocks.size(); ++k)
      for (auto &child : src.blocks[k]->ops) out->blocks[k]->ops.push_back(op(*child, out->blocks[k].get()));
    return out;
  }
};
} // namespace

std::unique_ptr<Module> cloneModule(const Module &module) {
  Cloner c;
  auto out = std::make_unique<Module>();
  out->op = c.op(*module.op, nullptr);
  return out;
}

std::unique_ptr<Op> cloneOp(const Op &op, Block *parent, ValueMap &map) {
  Cloner c{{}, map};
  return c.op(op, parent);
}

} // namespace ckl
