// Error reporting of the extern "C" surface: exceptions never cross the C-ABI;
// they become a non-zero tinymlp_last_error() and a message on stderr.
#pragma once

#include <cstdio>
#include <exception>
#include <string>

namespace graft {

void set_last_error(int code, const std::string& msg);

template <class F>
int guarded(const char* what, F&& f)
{
    try {
        f();
        set_last_error(0, std::string());
        return 0;
    } catch (const std::exception& e) {
        set_last_error(1, std::string(what) + ": " + e.what());
    } catch (...) {
        set_last_error(1, std::string(what) + ": unknown exception");
    }
    return 1;
}

}  // namespace graft
