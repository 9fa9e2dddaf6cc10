// sg_internal.h -- helpers shared by the library's host translation units.
#pragma once

namespace sgi {
// Records a printf-style message for sg_last_error() (thread-local) and
// returns `code`.
__attribute__((visibility("hidden"))) int fail(int code, const char* fmt, ...);
}  // namespace sgi
