/* Forwarding header: lets the reference's callers keep their
 * #include "tokenizer.h" (its include/tokenizer.h) and build against this library. */
#include "lunelette_tokenizer.h"
