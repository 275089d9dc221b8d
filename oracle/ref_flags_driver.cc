// ref_flags_driver.cc -- TEST INFRASTRUCTURE ONLY.
//
// Drives the reference's own flag parser, compiled unmodified from
// annc/service/cpu/annc_flags.cc (see oracle/Makefile), so tests can compare
// this library's ANNC_FLAGS parser against it.  Never linked into annc_amd.
#include <cstdlib>

#include "annc_flags.h"

// Returns 1 if `name` is enabled after the reference parses `flags` as the
// ANNC_FLAGS environment variable (annc_flags.cc:78-93: the constructor
// loads defaults, then parses the environment).
extern "C" int ref_flag_enabled(const char* flags, const char* name) {
  setenv("ANNC_FLAGS", flags, 1);
  annc::ANNCFlags parsed;
  return parsed.is_enabled(name) ? 1 : 0;
}
