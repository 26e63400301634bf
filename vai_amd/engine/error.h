// error.h -- VAI_ASSERT as the reference defines it (/root/reference/vai/engine/
// error.h:29-33, abort in debug, nothing under NDEBUG), plus the structural
// errors the engine throws as std::runtime_error (neural-net.cpp:341,353).
#pragma once
#include <cstdio>
#include <cstdlib>
#include <stdexcept>
#include <string>

#ifdef NDEBUG
#define VAI_ASSERT(cond) ((void)0)
#else
#define VAI_ASSERT(cond)                                                                             \
    do {                                                                                             \
        if (!(cond)) {                                                                               \
            std::fprintf(stderr, "VAI_ASSERT failed: %s (%s:%d)\n", #cond, __FILE__, __LINE__);       \
            std::abort();                                                                            \
        }                                                                                            \
    } while (0)
#endif

namespace vai {
// Shape / wiring checks that a caller can trigger with bad input: these throw
// in every build, so bindings and tests can observe them.
inline void require(bool cond, const std::string& what)
{
    if (!cond) throw std::runtime_error(what);
}
}   // namespace vai
