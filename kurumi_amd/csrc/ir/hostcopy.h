// Host-side bulk copies for tensors crossing the C boundary. One core copies fresh (never
// touched) memory at a few GB/s, most of it spent taking page faults, so GB-sized tensors are
// copied by several threads at once into destinations advised for transparent huge pages.
#pragma once
#include <cstddef>

namespace ku {

// Advise the kernel to back [p, p + n) with transparent huge pages on first touch (the 2 MiB
// aligned interior only). Best effort: errors are ignored. Call it on memory this library has
// just allocated and not yet written.
void advise_huge(void* p, size_t n);

// memcpy, split across up to `host_copy_threads()` threads when n is large. Returns after the
// whole copy is done.
void par_copy(void* dst, const void* src, size_t n);

// Threads par_copy uses for large copies: KURUMI_HOST_COPY_THREADS if set (1 disables the
// split), else min(8, hardware threads).
int host_copy_threads();

}  // namespace ku
