// dfattn_status.h — the library's error state, shared by every host-side
// source file (the state itself lives in dfattn_api.hip).
#pragma once

#include <string>

namespace dfattn {

// Records status and msg as the library's last error (dfattn_last_error,
// dfattn_last_error_message) and returns status.
int record_error(int status, const std::string &msg);

// For the reference launcher symbols (void return): keeps a failed status
// for darkforest_sync, which aborts on it.
void mark_pending(int status);

}  // namespace dfattn
