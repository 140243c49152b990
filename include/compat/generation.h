/* Forwarding header: lets the reference's callers keep their
 * #include "generation.h" (its include/generation.h) and build against this library. */
#include "lunelette_generation.h"
