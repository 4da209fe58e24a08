// qv_hip_util.hpp -- HIP error mapping and the C-ABI exception guard.
#pragma once

#include <hip/hip_runtime.h>

#include <exception>
#include <new>
#include <string>

#include "qv_common.hpp"

namespace qv {

inline void hip_check(hipError_t e, const char* what, const char* file, int line) {
  if (e == hipSuccess) return;
  const int code = (e == hipErrorOutOfMemory) ? QV_ENOMEM : QV_EHIP;
  fail(code, std::string(what) + " failed: " + hipGetErrorString(e) + " (" + file + ":" +
                 std::to_string(line) + ")");
}

#define HIP_OK(x) ::qv::hip_check((x), #x, __FILE__, __LINE__)

// Runs f, converting exceptions to a QV_* status and the thread-local message.
template <class F>
int guard(F&& f) {
  try {
    f();
    return QV_OK;
  } catch (const Error& e) {
    set_last_error(e.what());
    return e.code;
  } catch (const std::bad_alloc&) {
    set_last_error("host allocation failed");
    return QV_ENOMEM;
  } catch (const std::exception& e) {
    set_last_error(e.what());
    return QV_EIO;
  } catch (...) {
    set_last_error("unknown error");
    return QV_EIO;
  }
}

}  // namespace qv
