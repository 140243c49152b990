/* Forwarding header: lets the reference's callers keep their
 * #include "metal_weights.h" (its src/metal_weights.h) and build against this
 * library, which exports the caller-facing open/close of that header. */
#include "lunelette_runtime.h"
#include "lunelette_weights.h"
