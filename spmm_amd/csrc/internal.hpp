// Internal helpers shared by the translation units of libspmm_amd.so.
#pragma once

namespace spmm_internal {

// Records msg as this thread's spmm_last_error() and returns code.
__attribute__((visibility("hidden"))) int set_error(int code, const char* msg);

}  // namespace spmm_internal
