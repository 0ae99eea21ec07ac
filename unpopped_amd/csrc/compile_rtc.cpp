// The Compiler seam (trait Compiler, crates/unpopped/src/jit.rs:271-285) for gfx950: hipRTC,
// in process.  Artifacts are HIP code objects (ArtifactKind::HipCodeObject, jit.rs:144-145).
//
// Compiled modules are kept for the life of the process, keyed by the exact source text
// (compile once per source); nothing is written to disk and no prebuilt variant set ships.
#include <hip/hiprtc.h>

#include <chrono>
#include <map>
#include <mutex>

#include "unp_internal.hpp"

namespace unp {

namespace {

std::mutex g_mu;
std::map<std::string, std::vector<uint8_t>>& cache() {
  static std::map<std::string, std::vector<uint8_t>> c;
  return c;
}

// -ffp-contract=off: arithmetic is rounded as written (no fused multiply-add), as the
// reference's C leg compiles (crates/unpopped-cpu-c/tests/support/cc.rs:163-176).
// -packed-fp32-ops off: no v_pk_{add,mul,fma}_f32.
const char* const kOptions[] = {"--offload-arch=gfx950", "-O3",         "-std=c++17",
                                "-ffp-contract=off",     "-Xclang",     "-target-feature",
                                "-Xclang",               "-packed-fp32-ops"};

}  // namespace

int32_t compile_source(const std::string& source, const std::string& entry, uint32_t max_ms,
                       std::vector<uint8_t>& code, std::string& log) {
  {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = cache().find(source);
    if (it != cache().end()) {
      code = it->second;
      log.clear();
      return UNP_OK;
    }
  }
  const auto t0 = std::chrono::steady_clock::now();
  hiprtcProgram prog = nullptr;
  hiprtcResult r = hiprtcCreateProgram(&prog, source.c_str(), (entry + ".hip").c_str(), 0, nullptr, nullptr);
  if (r != HIPRTC_SUCCESS) {
    log = std::string("hiprtcCreateProgram: ") + hiprtcGetErrorString(r);
    return UNP_COMPILE_ERROR;
  }
  r = hiprtcCompileProgram(prog, (int)(sizeof(kOptions) / sizeof(kOptions[0])), kOptions);
  size_t log_size = 0;
  hiprtcGetProgramLogSize(prog, &log_size);
  log.assign(log_size, '\0');
  if (log_size) hiprtcGetProgramLog(prog, &log[0]);
  while (!log.empty() && log.back() == '\0') log.pop_back();
  if (r != HIPRTC_SUCCESS) {
    log = std::string("hiprtcCompileProgram: ") + hiprtcGetErrorString(r) + "\n" + log;
    hiprtcDestroyProgram(&prog);
    return UNP_COMPILE_ERROR;
  }
  size_t n = 0;
  hiprtcGetCodeSize(prog, &n);
  code.resize(n);
  hiprtcGetCode(prog, reinterpret_cast<char*>(code.data()));
  hiprtcDestroyProgram(&prog);
  const auto ms =
      std::chrono::duration_cast<std::chrono::milliseconds>(std::chrono::steady_clock::now() - t0).count();
  if (max_ms != 0 && ms > (long long)max_ms) {
    log = "compile took " + std::to_string(ms) + " ms, over the " + std::to_string(max_ms) + " ms budget";
    code.clear();
    return UNP_COMPILE_ERROR;
  }
  std::lock_guard<std::mutex> lk(g_mu);
  cache()[source] = code;
  return UNP_OK;
}

}  // namespace unp

extern "C" {

int32_t unp_hip_compile(const char* source, const char* entry, uint32_t max_compile_ms, uint8_t** bytes,
                        size_t* len, char** diag) {
  if (bytes) *bytes = nullptr;
  if (len) *len = 0;
  if (diag) *diag = nullptr;
  if (!source || !entry || !bytes || !len) return UNP_INVALID_ARGUMENT;
  std::vector<uint8_t> code;
  std::string log;
  const int32_t rc = unp::compile_source(source, entry, max_compile_ms, code, log);
  if (diag && !log.empty()) {
    *diag = static_cast<char*>(std::malloc(log.size() + 1));
    if (*diag) std::memcpy(*diag, log.c_str(), log.size() + 1);
  }
  if (rc != UNP_OK) return rc;
  *bytes = static_cast<uint8_t*>(std::malloc(code.size() ? code.size() : 1));
  if (!*bytes) return UNP_COMPILE_ERROR;
  std::memcpy(*bytes, code.data(), code.size());
  *len = code.size();
  return UNP_OK;
}

int32_t unp_hip_artifact_kind(void) { return UNP_ARTIFACT_HIP_CODE_OBJECT; }

void unp_free_bytes(uint8_t* p) { std::free(p); }
void unp_free_str(char* s) { std::free(s); }

}  // extern "C"
