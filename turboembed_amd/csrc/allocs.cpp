// The backend's heap allocations, counted where they happen: the library is
// linked with --wrap for malloc, calloc, realloc, aligned_alloc,
// posix_memalign and every global operator new, so each of those calls made
// by the backend's own code (its handles, vectors, strings and maps alike)
// comes here first, is counted for the process and for the calling thread,
// and goes on to the C library's or the C++ runtime's function. Calls made
// by other libraries (the HIP runtime, the host program) are not rewritten
// and not counted. A run reports the change of the calling thread's count
// across it, as the reference's counting allocator does for the core's
// allocations (core/tests/allocations.rs; core/cuda/backend.cpp:146-175).
#include <atomic>
#include <cstddef>
#include <cstdint>
#include <cstdlib>
#include <new>

namespace rocm {

std::atomic<uint64_t> host_allocs{0};
static thread_local uint64_t host_allocs_here = 0;

static inline void counted() {
    host_allocs.fetch_add(1, std::memory_order_relaxed);
    ++host_allocs_here;
}

uint64_t host_allocs_on_thread() { return host_allocs_here; }

}  // namespace rocm

extern "C" {

void *__real_malloc(size_t);
void *__real_calloc(size_t, size_t);
void *__real_realloc(void *, size_t);
void *__real_aligned_alloc(size_t, size_t);
int __real_posix_memalign(void **, size_t, size_t);
void *__real__Znwm(size_t);
void *__real__Znam(size_t);
void *__real__ZnwmRKSt9nothrow_t(size_t, const std::nothrow_t &);
void *__real__ZnamRKSt9nothrow_t(size_t, const std::nothrow_t &);
void *__real__ZnwmSt11align_val_t(size_t, std::align_val_t);
void *__real__ZnamSt11align_val_t(size_t, std::align_val_t);

__attribute__((visibility("hidden"))) void *__wrap_malloc(size_t n) {
    rocm::counted();
    return __real_malloc(n);
}
__attribute__((visibility("hidden"))) void *__wrap_calloc(size_t k, size_t n) {
    rocm::counted();
    return __real_calloc(k, n);
}
__attribute__((visibility("hidden"))) void *__wrap_realloc(void *p, size_t n) {
    rocm::counted();
    return __real_realloc(p, n);
}
__attribute__((visibility("hidden"))) void *__wrap_aligned_alloc(size_t a, size_t n) {
    rocm::counted();
    return __real_aligned_alloc(a, n);
}
__attribute__((visibility("hidden"))) int __wrap_posix_memalign(void **p, size_t a, size_t n) {
    rocm::counted();
    return __real_posix_memalign(p, a, n);
}
__attribute__((visibility("hidden"))) void *__wrap__Znwm(size_t n) {
    rocm::counted();
    return __real__Znwm(n);
}
__attribute__((visibility("hidden"))) void *__wrap__Znam(size_t n) {
    rocm::counted();
    return __real__Znam(n);
}
__attribute__((visibility("hidden"))) void *__wrap__ZnwmRKSt9nothrow_t(size_t n, const std::nothrow_t &t) {
    rocm::counted();
    return __real__ZnwmRKSt9nothrow_t(n, t);
}
__attribute__((visibility("hidden"))) void *__wrap__ZnamRKSt9nothrow_t(size_t n, const std::nothrow_t &t) {
    rocm::counted();
    return __real__ZnamRKSt9nothrow_t(n, t);
}
__attribute__((visibility("hidden"))) void *__wrap__ZnwmSt11align_val_t(size_t n, std::align_val_t a) {
    rocm::counted();
    return __real__ZnwmSt11align_val_t(n, a);
}
__attribute__((visibility("hidden"))) void *__wrap__ZnamSt11align_val_t(size_t n, std::align_val_t a) {
    rocm::counted();
    return __real__ZnamSt11align_val_t(n, a);
}

}  // extern "C"
