// Scope guard that brackets one kernel launch with HIP events when the
// library's profiler is enabled (see tgx_profile.cpp).
#pragma once

#include <hip/hip_runtime.h>

namespace tgx {

class ProfScope {
 public:
  ProfScope(const char* name, hipStream_t s);
  ~ProfScope();
  ProfScope(const ProfScope&) = delete;
  ProfScope& operator=(const ProfScope&) = delete;

 private:
  const char* name_;
  hipStream_t stream_;
  hipEvent_t start_ = nullptr;
};

}  // namespace tgx

#define TGX_PROF_CAT2(a, b) a##b
#define TGX_PROF_CAT(a, b) TGX_PROF_CAT2(a, b)
// Time the launch(es) issued in the rest of the enclosing block.
#define TGX_PROFILE(name, stream) \
  ::tgx::ProfScope TGX_PROF_CAT(tgx_prof_scope_, __LINE__)(name, stream)
