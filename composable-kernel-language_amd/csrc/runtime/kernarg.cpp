#include "kernarg.h"

#include <elf.h>

#include <cstring>
#include <memory>
#include <stdexcept>

namespace ckl::rt {
namespace {

[[noreturn]] void malformed(const char *what) {
  throw std::invalid_argument(std::string("code object metadata: ") + what);
}

// ------------------------------------------------------------------ MessagePack (the subset
// the AMDGPU metadata uses: maps, arrays, strings, integers, booleans, nil, floats, binary).
struct Node {
  enum Kind { Nil, Bool, Int, Float, Str, Bin, Array, Map } kind = Nil;
  int64_t integer = 0;
  std::string text;
  std::vector<Node> items;                       // Array: elements; Map: key, value, key, ...
  const Node *find(const char *key) const {
    if (kind != Map) return nullptr;
    for (size_t k = 0; k + 1 < items.size(); k += 2)
      if (items[k].kind == Str && items[k].text == key) return &items[k + 1];
    return nullptr;
  }
};

class Reader {
public:
  Reader(const uint8_t *data, size_t size) : p(data), end(data + size) {}

  Node value(int depth = 0) {
    if (depth > 32) malformed("nesting too deep");
    uint8_t tag = byte();
    Node n;
    if (tag <= 0x7f) { n.kind = Node::Int; n.integer = tag; return n; }
    if (tag >= 0xe0) { n.kind = Node::Int; n.integer = int8_t(tag); return n; }
    if ((tag & 0xf0) == 0x80) return container(Node::Map, tag & 0x0f, depth);
    if ((tag & 0xf0) == 0x90) return container(Node::Array, tag & 0x0f, depth);
    if ((tag & 0xe0) == 0xa0) return string(Node::Str, tag & 0x1f);
    switch (tag) {
    case 0xc0: return n;
    case 0xc2: case 0xc3: n.kind = Node::Bool; n.integer = tag == 0xc3; return n;
    case 0xc4: return string(Node::Bin, unsignedOf(1));
    case 0xc5: return string(Node::Bin, unsignedOf(2));
    case 0xc6: return string(Node::Bin, unsignedOf(4));
    case 0xca: skip(4); n.kind = Node::Float; return n;
    case 0xcb: skip(8); n.kind = Node::Float; return n;
    case 0xcc: n.kind = Node::Int; n.integer = int64_t(unsignedOf(1)); return n;
    case 0xcd: n.kind = Node::Int; n.integer = int64_t(unsignedOf(2)); return n;
    case 0xce: n.kind = Node::Int; n.integer = int64_t(unsignedOf(4)); return n;
    case 0xcf: n.kind = Node::Int; n.integer = int64_t(unsignedOf(8)); return n;
    case 0xd0: n.kind = Node::Int; n.integer = int8_t(unsignedOf(1)); return n;
    case 0xd1: n.kind = Node::Int; n.integer = int16_t(unsignedOf(2)); return n;
    case 0xd2: n.kind = Node::Int; n.integer = int32_t(unsignedOf(4)); return n;
    case 0xd3: n.kind = Node::Int; n.integer = int64_t(unsignedOf(8)); return n;
    case 0xd9: return string(Node::Str, unsignedOf(1));
    case 0xda: return string(Node::Str, unsignedOf(2));
    case 0xdb: return string(Node::Str, unsignedOf(4));
    case 0xdc: return container(Node::Array, unsignedOf(2), depth);
    case 0xdd: return container(Node::Array, unsignedOf(4), depth);
    case 0xde: return container(Node::Map, unsignedOf(2), depth);
    case 0xdf: return container(Node::Map, unsignedOf(4), depth);
    default: malformed("unsupported MessagePack tag");
    }
  }

private:
  const uint8_t *p, *end;

  uint8_t byte() {
    if (p >= end) malformed("truncated MessagePack");
    return *p++;
  }
  void skip(size_t n) {
    if (size_t(end - p) < n) malformed("truncated MessagePack");
    p += n;
  }
  uint64_t unsignedOf(int width) {   // big-endian
    uint64_t v = 0;
    for (int k = 0; k < width; ++k) v = (v << 8) | byte();
    return v;
  }
  Node string(Node::Kind kind, uint64_t length) {
    if (uint64_t(end - p) < length) malformed("truncated MessagePack string");
    Node n;
    n.kind = kind;
    n.text.assign(reinterpret_cast<const char *>(p), size_t(length));
    p += length;
    return n;
  }
  Node container(Node::Kind kind, uint64_t count, int depth) {
    if (count > uint64_t(end - p)) malformed("MessagePack container larger than its note");
    Node n;
    n.kind = kind;
    uint64_t entries = kind == Node::Map ? 2 * count : count;
    n.items.reserve(size_t(entries));
    for (uint64_t k = 0; k < entries; ++k) n.items.push_back(value(depth + 1));
    return n;
  }
};

// ------------------------------------------------------------------ containers
struct Span {
  const uint8_t *data;
  size_t size;
};

// The gfx950 code object inside an uncompressed clang offload bundle, or the image itself.
Span codeObject(const uint8_t *image, size_t bytes) {
  static const char kBundle[] = "__CLANG_OFFLOAD_BUNDLE__";
  const size_t magic = sizeof kBundle - 1;
  if (bytes < magic || std::memcmp(image, kBundle, magic) != 0) return {image, bytes};
  auto read64 = [&](size_t at) {
    if (at + 8 > bytes) malformed("truncated offload bundle");
    uint64_t v;
    std::memcpy(&v, image + at, 8);
    return v;
  };
  uint64_t count = read64(magic);
  size_t at = magic + 8;
  for (uint64_t k = 0; k < count; ++k) {
    uint64_t offset = read64(at), size = read64(at + 8), idSize = read64(at + 16);
    at += 24;
    if (idSize > bytes - at) malformed("truncated offload bundle entry");
    std::string id(reinterpret_cast<const char *>(image + at), size_t(idSize));
    at += size_t(idSize);
    if (id.find("amdgcn") != std::string::npos && id.find("gfx950") != std::string::npos) {
      if (offset > bytes || size > bytes - offset) malformed("offload bundle entry outside the image");
      return {image + offset, size_t(size)};
    }
  }
  malformed("offload bundle has no gfx950 code object");
}

Node metadataNote(Span elf) {
  if (elf.size < sizeof(Elf64_Ehdr)) malformed("image is not an ELF code object");
  Elf64_Ehdr header;
  std::memcpy(&header, elf.data, sizeof header);
  if (std::memcmp(header.e_ident, ELFMAG, SELFMAG) != 0 || header.e_ident[EI_CLASS] != ELFCLASS64)
    malformed("image is not a 64-bit ELF code object");
  if (header.e_shentsize != sizeof(Elf64_Shdr) || header.e_shoff > elf.size ||
      uint64_t(header.e_shnum) * sizeof(Elf64_Shdr) > elf.size - header.e_shoff)
    malformed("ELF section table outside the image");
  for (unsigned s = 0; s < header.e_shnum; ++s) {
    Elf64_Shdr section;
    std::memcpy(&section, elf.data + header.e_shoff + s * sizeof(Elf64_Shdr), sizeof section);
    if (section.sh_type != SHT_NOTE) continue;
    if (section.sh_offset > elf.size || section.sh_size > elf.size - section.sh_offset)
      malformed("ELF note section outside the image");
    const uint8_t *p = elf.data + section.sh_offset, *end = p + section.sh_size;
    while (size_t(end - p) >= sizeof(Elf64_Nhdr)) {
      Elf64_Nhdr note;
      std::memcpy(&note, p, sizeof note);
      p += sizeof note;
      size_t name = (size_t(note.n_namesz) + 3) & ~size_t(3), desc = (size_t(note.n_descsz) + 3) & ~size_t(3);
      if (name > size_t(end - p) || note.n_descsz > size_t(end - p) - name) malformed("truncated ELF note");
      bool amdgpu = note.n_namesz == 7 && std::memcmp(p, "AMDGPU", 7) == 0;
      if (amdgpu && note.n_type == 32 /* NT_AMDGPU_METADATA */)
        return Reader(p + name, note.n_descsz).value();
      p += name + std::min(desc, size_t(end - p) - name);
    }
  }
  malformed("no AMDGPU metadata note");
}

uint32_t field(const Node &map, const char *key) {
  const Node *v = map.find(key);
  if (!v || v->kind != Node::Int || v->integer < 0 || v->integer > 0xffffffffll)
    malformed((std::string("missing or invalid ") + key).c_str());
  return uint32_t(v->integer);
}

} // namespace

std::map<std::string, KernelSignature> readKernelSignatures(const void *image, size_t bytes) {
  if (!image || !bytes) malformed("empty image");
  Node root = metadataNote(codeObject(static_cast<const uint8_t *>(image), bytes));
  const Node *kernels = root.find("amdhsa.kernels");
  if (!kernels || kernels->kind != Node::Array) malformed("no amdhsa.kernels list");
  std::map<std::string, KernelSignature> out;
  for (const Node &kernel : kernels->items) {
    const Node *name = kernel.find(".name");
    if (!name || name->kind != Node::Str) malformed("kernel without a name");
    KernelSignature signature;
    signature.segmentBytes = field(kernel, ".kernarg_segment_size");
    if (const Node *args = kernel.find(".args")) {
      if (args->kind != Node::Array) malformed(".args is not a list");
      for (const Node &arg : args->items) {
        const Node *kind = arg.find(".value_kind");
        if (!kind || kind->kind != Node::Str) malformed("argument without a value kind");
        if (kind->text.rfind("hidden_", 0) == 0) continue;
        signature.arguments.push_back({field(arg, ".offset"), field(arg, ".size")});
      }
    }
    out[name->text] = std::move(signature);
  }
  return out;
}

} // namespace ckl::rt
