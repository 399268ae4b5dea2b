// trace.hpp -- leveled logging and roctx ranges.
//
// Reference counterparts (file:line in /root/reference):
//   logger, NVE_LOG_LEVEL   include/logging.hpp:34-203 (levels Critical 0,
//                           Error 10, Warning 20, Perf 30, Info 40, Verbose
//                           100; messages at or below the level are written,
//                           errors to stderr, the rest to stdout)
//   NVTX scoped ranges      include/cuda_support.hpp:26-55
//
// Here: one process-wide level, read from NVE_LOG_LEVEL (CRITICAL, ERROR,
// WARNING, PERF, INFO or VERBOSE; default WARNING) on first use and settable
// through the C ABI (nve_amd_set_log_level).  A message is formatted only when
// its level passes.  Scoped ranges are roctx ranges (rocprofv3 --marker-trace
// shows them); NVE_ROCTX=0 turns them off.
#pragma once

#include <stdint.h>

#include <sstream>
#include <string>

namespace nve_amd {

enum class LogLevel : int { Critical = 0, Error = 10, Warning = 20, Perf = 30, Info = 40, Verbose = 100 };

int log_level();
void set_log_level(int level);
bool log_enabled(LogLevel level);
void log_write(LogLevel level, const std::string& msg);
// the level named by s (the NVE_LOG_LEVEL names), or -1
int parse_log_level(const char* s);

template <typename... T>
void log_at(LogLevel level, const T&... parts) {
  if (!log_enabled(level)) return;
  std::ostringstream os;
  (os << ... << parts);
  log_write(level, os.str());
}

#define NVE_LOG_ERROR(...) ::nve_amd::log_at(::nve_amd::LogLevel::Error, __VA_ARGS__)
#define NVE_LOG_WARNING(...) ::nve_amd::log_at(::nve_amd::LogLevel::Warning, __VA_ARGS__)
#define NVE_LOG_PERF(...) ::nve_amd::log_at(::nve_amd::LogLevel::Perf, __VA_ARGS__)
#define NVE_LOG_INFO(...) ::nve_amd::log_at(::nve_amd::LogLevel::Info, __VA_ARGS__)
#define NVE_LOG_VERBOSE(...) ::nve_amd::log_at(::nve_amd::LogLevel::Verbose, __VA_ARGS__)

// roctx range for the scope: pushed at construction, popped at destruction
class TraceRange {
 public:
  explicit TraceRange(const char* name);
  ~TraceRange();
  TraceRange(const TraceRange&) = delete;
  TraceRange& operator=(const TraceRange&) = delete;

 private:
  bool on_;
};

#define NVE_TRACE_CAT2(a, b) a##b
#define NVE_TRACE_CAT(a, b) NVE_TRACE_CAT2(a, b)
#define NVE_TRACE(name) ::nve_amd::TraceRange NVE_TRACE_CAT(nve_trace_, __LINE__)(name)

}  // namespace nve_amd
