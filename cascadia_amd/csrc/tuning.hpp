// tuning.hpp -- the CASCADIA_INT4_* tuning variables (plan overrides), read
// once per process.
#pragma once

namespace cai4 {

// The environment variable `name` as an int, or `absent` when it is unset or
// does not start with a number.  Each name is read from the environment once
// and cached; cascadia_int4_reload_tuning() drops the cache so the next call
// reads the environment again.  `name` must be a string literal.
int tuning_env(const char *name, int absent);

}  // namespace cai4
