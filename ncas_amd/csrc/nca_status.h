// The library's error channel (thread-local message read by nca_last_error), shared by the
// translation units of libnca_hip.so.
#pragma once

#include <hip/hip_runtime.h>

namespace nca {

int set_error(int code, const char *msg);           // stores msg, returns code
void clear_error();                                  // empties the message (start of an entry point)
int hip_status(hipError_t e, const char *what);      // NCA_OK, or NCA_ERR_HIP with the HIP message

}  // namespace nca
