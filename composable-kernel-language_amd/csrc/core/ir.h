// CKL kernel/program IR: an MLIR-compatible textual subset, parsed and printed without MLIR.
//
// The frontend (python/ckl/frontend/emitter.py) prints programs in this syntax; the
// analyses in analysis.cpp read them. Ops keep MLIR's generic structure (name, operands,
// results, attributes, regions) so that the same walk order, SSA identity and attribute
// names used by the reference passes (lib/Analysis/GraphAnalysis.cpp,
// lib/Analysis/EffectAnalysis.cpp) carry over to this implementation.
#pragma once

#include <cstdint>
#include <functional>
#include <map>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

namespace ckl {

struct IRError : std::runtime_error {
  using std::runtime_error::runtime_error;
};

// ---------------------------------------------------------------- types
struct Type {
  enum Kind { None, F16, F32, F64, I1, I8, I32, I64, Index, MemRef, Token, Vector, Opaque };
  Kind kind = None;
  Kind element = None;            // memref / vector element kind
  std::vector<int64_t> shape;     // -1 = dynamic extent
  bool unranked = false;          // memref<*xT>
  bool identityLayout = true;     // false for strided<...> / affine_map<...> layouts
  std::string layout;             // spelling of a non-identity layout, empty = identity
  std::string memorySpace;        // empty = default (global)
  std::string text;               // opaque spelling

  static Type scalar(Kind k) { Type t; t.kind = k; return t; }
  static Type memref(Kind elem, std::vector<int64_t> shape) {
    Type t; t.kind = MemRef; t.element = elem; t.shape = std::move(shape); return t;
  }
  bool isMemRef() const { return kind == MemRef; }
  bool isFloat() const { return kind == F16 || kind == F32 || kind == F64; }
  bool isInteger() const { return kind == I1 || kind == I8 || kind == I32 || kind == I64; }
  bool isIntOrIndex() const { return isInteger() || kind == Index; }
  bool hasStaticShape() const;
  // Element width in bits for scalars (index = 64) and memref/vector elements.
  static unsigned bitWidth(Kind k);
  int64_t elementCount() const;   // -1 when not static
  std::string str() const;
  bool operator==(const Type &o) const { return str() == o.str(); }
  bool operator!=(const Type &o) const { return !(*this == o); }
};

std::string kindName(Type::Kind k);

// ---------------------------------------------------------------- attributes
struct Attr {
  enum Kind { Null, Int, Float, String, Bool, Unit, Array, DenseI64, DenseI32, DenseI8, Symbol, Dict, TypeAttr };
  Kind kind = Null;
  int64_t i = 0;
  double f = 0;
  std::string s;                                  // string / symbol (root name, no '@')
  std::vector<std::string> nested;                // nested symbol path after the root
  Type type;                                      // int/float element type or TypeAttr value
  std::vector<Attr> array;                        // Array
  std::vector<int64_t> dense;                     // DenseI64/I32/I8
  std::vector<std::pair<std::string, Attr>> dict; // Dict, sorted by key

  static Attr integer(int64_t v, Type::Kind t = Type::I64) { Attr a; a.kind = Int; a.i = v; a.type = Type::scalar(t); return a; }
  static Attr floating(double v, Type::Kind t) { Attr a; a.kind = Float; a.f = v; a.type = Type::scalar(t); return a; }
  static Attr string(std::string v) { Attr a; a.kind = String; a.s = std::move(v); return a; }
  static Attr boolean(bool v) { Attr a; a.kind = Bool; a.i = v; return a; }
  static Attr unit() { Attr a; a.kind = Unit; return a; }
  static Attr arrayOf(std::vector<Attr> v) { Attr a; a.kind = Array; a.array = std::move(v); return a; }
  static Attr denseI64(std::vector<int64_t> v) { Attr a; a.kind = DenseI64; a.dense = std::move(v); return a; }
  static Attr denseI32(std::vector<int64_t> v) { Attr a; a.kind = DenseI32; a.dense = std::move(v); return a; }
  static Attr symbol(std::string v) { Attr a; a.kind = Symbol; a.s = std::move(v); return a; }
  static Attr typeAttr(Type t) { Attr a; a.kind = TypeAttr; a.type = std::move(t); return a; }
  static Attr dictOf(std::vector<std::pair<std::string, Attr>> entries);

  bool isNull() const { return kind == Null; }
  const Attr *get(const std::string &key) const;   // Dict lookup
  std::string str() const;
  bool operator==(const Attr &o) const { return str() == o.str(); }
  bool operator!=(const Attr &o) const { return !(*this == o); }
};

// ---------------------------------------------------------------- operations
struct Op;
struct Block;
struct Region;

struct Value {
  Type type;
  Op *def = nullptr;        // defining op, or null for a block argument
  Block *owner = nullptr;   // owning block for block arguments
  unsigned index = 0;       // result number or argument number
  std::string hint;         // source spelling (without '%'), informational only
};

struct Block {
  std::vector<std::unique_ptr<Value>> args;
  std::vector<std::unique_ptr<Op>> ops;
  Region *parent = nullptr;
};

struct Region {
  std::vector<std::unique_ptr<Block>> blocks;
  Op *parent = nullptr;
};

struct Op {
  std::string name;
  std::vector<Value *> operands;
  std::vector<std::unique_ptr<Value>> results;
  std::map<std::string, Attr> attrs;
  std::vector<std::unique_ptr<Region>> regions;
  Block *parent = nullptr;
  std::string loc;          // printed location, e.g. "file.py":12:3, empty = unknown
  unsigned line = 0, column = 0;   // position in the parsed text (1-based), 0 = not parsed

  const Attr *attr(const std::string &key) const {
    auto it = attrs.find(key);
    return it == attrs.end() ? nullptr : &it->second;
  }
  Value *result(unsigned i = 0) const { return results.at(i).get(); }
  Op *parentOp() const;
  // Func helpers (name == "func.func")
  std::string symName() const;
  Block *entry() const;
  bool isDeclaration() const { return regions.empty() || regions[0]->blocks.empty(); }
};

struct Module {
  std::unique_ptr<Op> op;   // builtin.module
  std::vector<Op *> functions() const;
  Op *lookup(const std::string &symbol) const;
  Block *body() const { return op->regions[0]->blocks[0].get(); }
};

// Parse an MLIR-syntax module subset (generic ops plus the func/arith/math/scf/memref
// pretty forms that the frontend emits). Throws IRError with "line:col: message".
std::unique_ptr<Module> parseModule(const std::string &text);

// Printing. `locations` adds loc(...) suffixes. Value names are renumbered canonically
// (%arg0.., %0..) so equal IR prints equal text regardless of source spelling.
std::string printModule(const Module &module, bool locations = false);
std::string printOp(const Op &op, bool locations = false, int indent = 0);
// Canonical text of a function body and signature with the symbol name omitted.
std::string canonicalFunction(const Op &function);

// Deep copy (values remapped).
std::unique_ptr<Module> cloneModule(const Module &module);
// Copy of `op` (with its regions) owned by `parent`: operands found in `map` are replaced, and
// the copies of results and block arguments are recorded in `map`.
using ValueMap = std::unordered_map<const Value *, Value *>;
std::unique_ptr<Op> cloneOp(const Op &op, Block *parent, ValueMap &map);

// Diagnostic prefix naming where an op came from: its loc(...) when it has one, else its
// "line:col" in the parsed text, followed by ": "; empty when neither is known.
std::string sourcePosition(const Op *op);

// Walk helpers.
void walkPreOrder(Op *op, const std::function<void(Op *)> &fn);

} // namespace ckl
