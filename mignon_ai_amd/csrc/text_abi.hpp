// Shared by the library's translation units: the thread-local message mg_last_error() returns.
#pragma once

#include <string>

struct mg_model;
struct mg_sessions;

namespace mg {
void set_last_error(const std::string& msg);

// The session set mg_generate_greedy and mg_generate_sample decode on: the one the model kept from its
// last generate call when that has n sessions and the same window (its state cleared as a new set's),
// else a new set. Returns an MG_* code. Hand the set back with generate_sessions_release, which keeps it
// in the model (freed with the model, or when a later call needs another size).
int generate_sessions_acquire(mg_model* m, int n, int context, mg_sessions** out);
void generate_sessions_release(mg_model* m, mg_sessions* s);
}  // namespace mg
