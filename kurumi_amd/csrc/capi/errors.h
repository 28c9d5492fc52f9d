// The C ABI's thread-local last error (kurumi/src/capi.rs:24-60 analog), shared by the
// translation units that implement entry points.
#pragma once
#include <exception>
#include <string>

namespace ku::capi {

void set_err(const std::string& m);

// Run `f`, turning any exception into the last error and the failure value `fail`.
template <class R, class F>
R guard(R fail, F&& f) {
  try {
    return f();
  } catch (const std::exception& e) {
    set_err(e.what());
  } catch (...) {
    set_err("unknown error");
  }
  return fail;
}

}  // namespace ku::capi
