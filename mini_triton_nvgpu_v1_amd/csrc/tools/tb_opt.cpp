// tb-opt: the plan-pipeline driver (reference tools/tb-opt.cpp:11-24, an
// MlirOptMain over the tb passes). Reads textual IR, runs the passes named
// by --pass-pipeline or by individual --<pass>[=<options>] flags in command
// line order, and prints the resulting IR.
//
//   tb-opt in.mlir --pass-pipeline='builtin.module(tb-stage1-full-to-gfx950-pipeline{cubin-chip=gfx950})' -o out.mlir
//   tb-opt in.mlir --tb-verify-scope --tb-attach-target-info='gpu-arch=gfx950'
//
// Diagnostics go to stderr as `<file>: error: <message>` with exit code 1.
#include "../passes/passes.h"
#include "../plan/instances.h"

#include <cstdio>
#include <cstring>
#include <fstream>
#include <iostream>
#include <sstream>

namespace {

std::string readAll(const std::string &path) {
  if (path == "-") {
    std::ostringstream ss;
    ss << std::cin.rdbuf();
    return ss.str();
  }
  std::ifstream in(path, std::ios::binary);
  if (!in)
    throw tb::Error("cannot open `" + path + "`");
  std::ostringstream ss;
  ss << in.rdbuf();
  return ss.str();
}

void usage() {
  std::printf("usage: tb-opt [input.mlir|-] [-o output] "
              "[--pass-pipeline='builtin.module(...)'] [--<pass>[=<options>]]...\n"
              "       tb-opt --list-passes\n"
              "       tb-opt --list-instances   (the gfx950 kernels a plan can bind, with the\n"
              "                                  issue schedule and waits the plan states and\n"
              "                                  the compiled registers and scratch bytes)\n");
}

} // namespace

int main(int argc, char **argv) {
  std::string input = "-", output = "-";
  std::vector<tb::PassSpec> passes;
  try {
    for (int i = 1; i < argc; ++i) {
      std::string a = argv[i];
      if (a == "-h" || a == "--help") {
        usage();
        return 0;
      }
      if (a == "--list-passes") {
        for (const tb::PassInfo &p : tb::registeredPasses())
          std::printf("%-40s %s\n", p.name.c_str(), p.summary.c_str());
        return 0;
      }
      if (a == "--list-instances") {
        // name, the s_waitcnt depths the plan states for it, and the
        // compiler's register and scratch report of its build
        for (const tb::InstanceKey &k : tb::gfx950Instances()) {
          const tb::InstanceSchedule s = tb::instanceSchedule(k);
          const tb::InstanceResources r = tb::instanceResources(k);
          const tb::InstanceResources rk = tb::instanceResources(k, true);
          std::printf("%s %s vmcnt_prologue=%lld vmcnt_loop=%lld lgkmcnt_loop=%lld "
                      "loader_waves=%lld vgprs=%lld agprs=%lld scratch=%lld "
                      "scratch_partial_k=%lld\n",
                      tb::instanceName(k).c_str(), s.issue.c_str(), (long long)s.vmPrologue,
                      (long long)s.vmLoop, (long long)s.lgkmLoop, (long long)s.loaderWaves,
                      (long long)r.vgprs, (long long)r.agprs,
                      r.known ? (long long)r.scratchBytes : -1LL,
                      rk.known ? (long long)rk.scratchBytes : -1LL);
        }
        return 0;
      }
      if (a == "-o") {
        if (++i >= argc)
          throw tb::Error("-o needs a path");
        output = argv[i];
      } else if (a.rfind("--pass-pipeline=", 0) == 0) {
        for (tb::PassSpec &p : tb::parsePassPipeline(a.substr(16)))
          passes.push_back(p);
      } else if (a == "--pass-pipeline") {
        if (++i >= argc)
          throw tb::Error("--pass-pipeline needs a value");
        for (tb::PassSpec &p : tb::parsePassPipeline(argv[i]))
          passes.push_back(p);
      } else if (a.rfind("--tb-", 0) == 0) {
        std::string body = a.substr(2);
        size_t eq = body.find('=');
        std::string spec = eq == std::string::npos
                               ? body
                               : body.substr(0, eq) + "{" + body.substr(eq + 1) + "}";
        for (tb::PassSpec &p : tb::parsePassPipeline(spec))
          passes.push_back(p);
      } else if (!a.empty() && a[0] == '-' && a != "-") {
        throw tb::Error("unknown option `" + a + "`");
      } else {
        input = a;
      }
    }
  } catch (const tb::Error &e) {
    std::fprintf(stderr, "tb-opt: error: %s\n", e.what());
    return 1;
  }
  try {
    tb::Module m = tb::parseModule(readAll(input));
    tb::runPipeline(m, passes);
    std::string text = tb::printModule(m);
    if (output == "-") {
      std::fwrite(text.data(), 1, text.size(), stdout);
    } else {
      std::ofstream out(output, std::ios::binary);
      if (!out)
        throw tb::Error("cannot write `" + output + "`");
      out << text;
    }
  } catch (const tb::Error &e) {
    std::fprintf(stderr, "%s: error: %s\n", input.c_str(), e.what());
    return 1;
  }
  return 0;
}
