// No C++ exception crosses the C ABI: the entry points that allocate host
// memory (std::vector, std::string, std::thread) run their body through
// guarded(), which turns an exception into the entry point's failure value
// (-1 or NULL) with the reason in the context's error string.
#pragma once

#include <cstdio>
#include <exception>
#include <new>
#include <string>
#include <type_traits>

namespace tpmd {

template <typename Ctx, typename F>
auto guarded(Ctx *c, F &&body) -> decltype(body()) {
    using R = decltype(body());
    const char *what = "internal error";
    std::string msg;
    try {
        return body();
    } catch (const std::bad_alloc &) {
        what = "out of host memory";
    } catch (const std::exception &e) {
        try {
            msg = std::string("internal error: ") + e.what();
            what = msg.c_str();
        } catch (...) {
        }
    } catch (...) {
    }
    if constexpr (std::is_same_v<Ctx, void>) {
        fprintf(stderr, "%s\n", what);
    } else if (c) {
        try {
            c->err = what;
        } catch (...) {
        }
    }
    if constexpr (std::is_pointer_v<R>)
        return nullptr;
    else
        return (R) -1;
}

}  // namespace tpmd
