// trace.cpp -- process-wide log level and writer, roctx ranges.
#include "trace.hpp"

#include <rocprofiler-sdk-roctx/roctx.h>

#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <ctime>
#include <mutex>

namespace nve_amd {

namespace {

struct Named {
  const char* name;
  LogLevel level;
};
constexpr Named kLevels[] = {{"CRITICAL", LogLevel::Critical}, {"ERROR", LogLevel::Error},
                             {"WARNING", LogLevel::Warning},   {"PERF", LogLevel::Perf},
                             {"INFO", LogLevel::Info},         {"VERBOSE", LogLevel::Verbose}};

char level_letter(LogLevel l) {
  switch (l) {
    case LogLevel::Critical: return 'C';
    case LogLevel::Error: return 'E';
    case LogLevel::Warning: return 'W';
    case LogLevel::Perf: return 'P';
    case LogLevel::Info: return 'I';
    case LogLevel::Verbose: return 'V';
  }
  return '?';
}

std::atomic<int>& level_ref() {
  static std::atomic<int> level{[] {
    const char* env = std::getenv("NVE_LOG_LEVEL");
    if (env == nullptr || *env == '\0') return (int)LogLevel::Warning;
    const int parsed = parse_log_level(env);
    if (parsed >= 0) return parsed;
    std::fprintf(stderr, "[NVE][W] NVE_LOG_LEVEL=%s is not a level name; using WARNING\n", env);
    return (int)LogLevel::Warning;
  }()};
  return level;
}

bool roctx_on() {
  static const bool on = [] {
    const char* env = std::getenv("NVE_ROCTX");
    return env == nullptr || std::strcmp(env, "0") != 0;
  }();
  return on;
}

std::mutex& write_mu() {
  static std::mutex mu;
  return mu;
}

}  // namespace

int parse_log_level(const char* s) {
  if (s == nullptr) return -1;
  for (const Named& n : kLevels)
    if (std::strcmp(s, n.name) == 0) return (int)n.level;
  return -1;
}

int log_level() { return level_ref().load(std::memory_order_relaxed); }

void set_log_level(int level) { level_ref().store(level, std::memory_order_relaxed); }

bool log_enabled(LogLevel level) { return (int)level <= log_level(); }

void log_write(LogLevel level, const std::string& msg) {
  const auto now = std::chrono::system_clock::now();
  const std::time_t t = std::chrono::system_clock::to_time_t(now);
  const long us = (long)(std::chrono::duration_cast<std::chrono::microseconds>(now.time_since_epoch())
                             .count() %
                         1000000);
  std::tm tm{};
  localtime_r(&t, &tm);
  char stamp[32];
  std::strftime(stamp, sizeof stamp, "%H:%M:%S", &tm);
  std::lock_guard<std::mutex> lk(write_mu());
  std::FILE* f = (int)level <= (int)LogLevel::Error ? stderr : stdout;
  std::fprintf(f, "[NVE %s.%06ld][%c] %s\n", stamp, us, level_letter(level), msg.c_str());
  std::fflush(f);
}

TraceRange::TraceRange(const char* name) : on_(roctx_on()) {
  if (on_) roctxRangePushA(name);
}

TraceRange::~TraceRange() {
  if (on_) roctxRangePop();
}

}  // namespace nve_amd
