// rxmet_error.cpp — error state and version of the rxmet C ABI.
#include <string>

#include "rxmet_common.h"

namespace rxmet {

static thread_local std::string g_last_error;

void set_error(const std::string &msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

}  // namespace rxmet

extern "C" {

const char *rxmet_last_error(void) { return rxmet::g_last_error.c_str(); }

int rxmet_abi_version(void) { return 1; }

}  // extern "C"
