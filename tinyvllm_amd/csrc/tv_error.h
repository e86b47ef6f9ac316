// Error reporting shared by the C-ABI translation units: a failing entry point
// records a message (thread-local) and returns a TV_E* code.
#pragma once

namespace tv {

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int ok();
int check_launch(const char* what);   // TV_EHIP if the last launch failed, else TV_OK
const char* last_error();

}  // namespace tv
