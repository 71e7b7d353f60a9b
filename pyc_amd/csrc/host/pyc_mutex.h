/* pyc_mutex.h — statically initialisable process-wide mutex for the engine's
 * global tables (registry, compile cache, GPU workspace). Same role as the
 * reference's include/pyc/pyc_mutex.h; POSIX only on this build. */
#ifndef PYC_AMD_MUTEX_H
#define PYC_AMD_MUTEX_H

#include <pthread.h>

typedef pthread_mutex_t pyc_mutex;
#define PYC_MUTEX_INIT PTHREAD_MUTEX_INITIALIZER

static inline void pyc_mutex_lock(pyc_mutex* m) { pthread_mutex_lock(m); }
static inline void pyc_mutex_unlock(pyc_mutex* m) { pthread_mutex_unlock(m); }

#endif
