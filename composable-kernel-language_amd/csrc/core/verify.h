// Verification of parsed CKL IR and reading of textual executable plans.
//
// Every module the pass driver reads is verified before any pass runs, as an MLIR tool verifies
// what it parses. The rules are those of the ckl dialect's operations and of the ckl.kernel
// function attribute (lib/Dialect/CKL/IR/CKLOps.cpp:17-207, lib/Dialect/CKL/IR/CKLDialect.cpp:19-35)
// and of the executable-plan operations (lib/Dialect/Exec/IR/CKLExecOps.cpp:35-192; the checks
// themselves are ExecPlan::verify in analysis.cpp). Diagnostics name the op and its position:
//   "12:5: 'ckl.dispatch' op requires positive block dimensions"
#pragma once

#include "analysis.h"

#include <vector>

namespace ckl {

struct VerifyOptions {
  // Accept operations of dialects this build does not know (--allow-unregistered-dialect).
  bool allowUnregisteredDialects = false;
};

// Throws CompileError on the first rule an operation breaks.
void verifyModule(const Module &module, const VerifyOptions &options = {});

// The executable plans written as "ckl_exec.plan" operations at module level, in order, each
// read back into plan form and verified.
std::vector<ExecPlan> readExecPlans(const Module &module);

} // namespace ckl
