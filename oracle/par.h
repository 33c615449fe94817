/* par.h — a parallel-for over index ranges with pthreads, for the oracle's CPU-baseline timings (the reference
 * parallelises the same loops with rayon: par_rows, tensor.rs:678-698; QuantAct::from_rows, packed.rs:389-419;
 * linear, tensor.rs:115-126; the attention tasks, encoder.rs:457-533). Outputs of different indices are disjoint,
 * so results do not depend on the thread count. TEST INFRASTRUCTURE ONLY. */
#ifndef VOXRT_ORACLE_PAR_H
#define VOXRT_ORACLE_PAR_H
#include <pthread.h>
#include <stddef.h>

typedef void (*or_range_fn)(void *ctx, size_t lo, size_t hi);

int or_get_threads(void);
void or_set_threads(int n);
void or_par_for(size_t n, or_range_fn fn, void *ctx);

#endif
