// Error plumbing for the C ABI: C++ code throws st::Error, every extern "C"
// entry point converts it into a status code plus a thread-local message.
#pragma once

#include <sstream>
#include <stdexcept>
#include <string>

#include "../../include/silvertorch_hip.h"

namespace st {

struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

void set_last_error(const std::string& msg);

template <typename... Args>
std::string cat(const Args&... args) {
  std::ostringstream os;
  (os << ... << args);
  return os.str();
}

template <typename... Args>
[[noreturn]] void fail(const Args&... args) {
  throw Error(ST_ERR_INVALID_ARGUMENT, cat(args...));
}

#define ST_CHECK(cond, ...)                                    \
  do {                                                         \
    if (!(cond)) ::st::fail(__VA_ARGS__);                      \
  } while (0)

// Runs `body` and maps exceptions onto the C status convention.
template <typename F>
int guarded(F&& body) {
  try {
    body();
    return ST_OK;
  } catch (const Error& e) {
    set_last_error(e.what());
    return e.code;
  } catch (const std::bad_alloc&) {
    set_last_error("host allocation failed");
    return ST_ERR_INVALID_ARGUMENT;
  } catch (const std::exception& e) {
    set_last_error(e.what());
    return ST_ERR_INVALID_ARGUMENT;
  }
}

}  // namespace st
