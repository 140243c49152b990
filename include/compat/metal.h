/* Forwarding header: lets the reference's callers keep their
 * #include "metal.h" (its include/metal.h) and build against this library. */
#include "lunelette_runtime.h"
