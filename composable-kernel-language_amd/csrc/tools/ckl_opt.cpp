// ckl-opt: command-line driver for the CKL pass pipeline (the reference's MlirOptMain-based
// tools/ckl-opt/ckl-opt.cpp:1-29, with the flag spellings its tests use).
//
//   ckl-opt <input | -> [--allow-unregistered-dialect] [--ckl-<pass>[=<option>,...]]... [-o <file>]
//
// Reads IR text from a file or stdin, verifies it, runs the passes in command-line order and
// prints the resulting module; with no pass it prints the verified module. On a parse, verify or
// pass error it prints "<input>:<line>:<col>: error: <message>" (position when known) on stderr
// and exits with status 1; bad usage exits with status 2. Everything runs through the C ABI's
// ckl_opt entry of libckl_hip.so, so the tool and the library accept exactly the same IR.
#include "../../../include/ckl_hip.h"

#include <cctype>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <iostream>
#include <iterator>
#include <sstream>
#include <string>
#include <vector>

namespace {

const char *kUsage =
    "usage: ckl-opt <input.mlir | -> [options]\n"
    "  --allow-unregistered-dialect      accept operations of dialects this build does not know\n"
    "  --ckl-summarize-effects[=strict=false]\n"
    "                                    attach ckl.effect_summary to every function\n"
    "  --ckl-build-graph[=strict=false,reuse-storage=false]\n"
    "                                    dependency graph, resources and memory plan per host function\n"
    "  --ckl-lower-graph-to-exec         lower the graphs to executable plans (ckl_exec.plan)\n"
    "  --ckl-prepare-hip                 validate kernels and assign HIP launch and artifact identities\n"
    "  --ckl-fuse-pointwise              guarded unary pointwise fusion\n"
    "  --ckl-lower-exec-to-host          the native host entry's callback sequence (last pass)\n"
    "  -o <file>                         write the output to <file> instead of stdout\n";

const char *kPasses[] = {"summarize-effects", "build-graph", "lower-graph-to-exec", "prepare-hip", "fuse-pointwise",
                         "lower-exec-to-host"};

// "--ckl-build-graph=strict=false,reuse-storage=false" -> "build-graph{strict=false,reuse-storage=false}".
bool passSpec(const std::string &flag, std::string &spec) {
  if (flag.rfind("--ckl-", 0) != 0) return false;
  std::string body = flag.substr(6);
  size_t eq = body.find('=');
  std::string name = body.substr(0, eq);
  bool known = false;
  for (const char *p : kPasses) known |= name == p;
  if (!known) return false;
  spec = eq == std::string::npos ? name : name + "{" + body.substr(eq + 1) + "}";
  return true;
}

// "12:5: message" -> ("12:5", "message"); other messages have no position.
std::pair<std::string, std::string> splitPosition(const std::string &message) {
  size_t k = 0;
  while (k < message.size() && std::isdigit((unsigned char)message[k])) ++k;
  if (k == 0 || k >= message.size() || message[k] != ':') return {"", message};
  size_t j = k + 1;
  while (j < message.size() && std::isdigit((unsigned char)message[j])) ++j;
  if (j == k + 1 || message.compare(j, 2, ": ") != 0) return {"", message};
  return {message.substr(0, j), message.substr(j + 2)};
}

} // namespace

int main(int argc, char **argv) {
  std::string input, output;
  std::vector<std::string> passes;
  for (int k = 1; k < argc; ++k) {
    std::string arg = argv[k], spec;
    if (arg == "-h" || arg == "--help") {
      std::fputs(kUsage, stdout);
      return 0;
    } else if (arg == "--allow-unregistered-dialect") {
      passes.push_back("allow-unregistered-dialect");
    } else if (passSpec(arg, spec)) {
      passes.push_back(spec);
    } else if (arg == "-o" && k + 1 < argc) {
      output = argv[++k];
    } else if (arg.rfind("-o", 0) == 0 && arg.size() > 2 && arg[2] != '-') {
      output = arg.substr(2);
    } else if ((arg == "-" || arg[0] != '-') && input.empty()) {
      input = arg;
    } else {
      std::fprintf(stderr, "ckl-opt: unknown argument '%s'\n%s", arg.c_str(), kUsage);
      return 2;
    }
  }
  if (input.empty()) input = "-";

  std::string text;
  if (input == "-") {
    text.assign(std::istreambuf_iterator<char>(std::cin), std::istreambuf_iterator<char>());
  } else {
    std::ifstream file(input, std::ios::binary);
    if (!file) {
      std::fprintf(stderr, "ckl-opt: cannot open input file '%s'\n", input.c_str());
      return 1;
    }
    text.assign(std::istreambuf_iterator<char>(file), std::istreambuf_iterator<char>());
  }

  std::string joined;
  for (size_t k = 0; k < passes.size(); ++k) joined += (k ? ";" : "") + passes[k];
  char *result = nullptr;
  if (ckl_opt(text.c_str(), joined.c_str(), &result) != 0) {
    auto [position, message] = splitPosition(ckl_last_error());
    std::string where = input == "-" ? "<stdin>" : input;
    if (!position.empty()) where += ":" + position;
    std::fprintf(stderr, "%s: error: %s\n", where.c_str(), message.c_str());
    return 1;
  }
  std::string out = result;
  ckl_string_free(result);
  if (output.empty() || output == "-") {
    std::fwrite(out.data(), 1, out.size(), stdout);
  } else {
    std::ofstream file(output, std::ios::binary);
    if (!(file << out)) {
      std::fprintf(stderr, "ckl-opt: cannot write '%s'\n", output.c_str());
      return 1;
    }
  }
  return 0;
}
