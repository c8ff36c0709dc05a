// Thread-local error message shared by every translation unit of libckv_amd.so.
#pragma once

namespace ckv_internal {
// Records `message` for ckv_last_error() and returns `code`.
int set_error(int code, const char* message);
}  // namespace ckv_internal
