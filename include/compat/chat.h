/* Forwarding header: lets the reference's callers keep their
 * #include "chat.h" (its include/chat.h) and build against this library. */
#include "lunelette_chat.h"
