// hh_host.h — host-side helpers shared by the library's translation units.
#pragma once
#include <string>

// Record msg as the calling thread's hh_last_error() and return code.
int hh_set_error(int code, const std::string& msg);
