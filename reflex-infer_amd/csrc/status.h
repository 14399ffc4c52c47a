// status.h -- the thread-local "last error" of the C ABI (rxq4_last_error),
// shared by the entry points in other translation units.
#pragma once

namespace rxq4 {

// Records the formatted reason and returns `status`.
int set_error(int status, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the reason and returns RXQ4_STATUS_SUCCESS.
int set_ok();

}  // namespace rxq4
