/* Native session adapter over the runtime C-ABI (include/lunelette_runtime.h).
 *
 * Replaces the model-facing half of the reference's native service adapter,
 * service/native.c: the chunked materialization state machine with the three
 * prefix-reuse policies (service/native.c:161-264), checkpoint save/restore
 * (:266-327), greedy or forced selection with the LNRPLY1 replay capture
 * (:336-416) and the option admission and memory/strategy checks at open
 * (:431-560). The tokenizer callbacks of service_generator (frame, piece,
 * tool_frame) and the file hashing of the service identity are not part of
 * this library: the service binds them beside these entry points.
 *
 * Return conventions follow service/session.h:31, 50-67: materialize returns
 * 0 (rejected or failed), 1 (ready) or LUNELETTE_SESSION_MORE (one block
 * committed, more to ingest); save/restore return 1 (done), 0 (rejected
 * before any change) or -1 (recovery required); next/replay_next return the
 * selected token (EOS 2 included) or -1 without publishing a pending token.
 *
 * One caller per session; the session owns its runtime and destroys it.
 */
#ifndef LUNELETTE_SESSION_H
#define LUNELETTE_SESSION_H

#include <stddef.h>
#include <stdint.h>

#include "lunelette_runtime.h"

#ifdef __cplusplus
extern "C" {
#endif

#define LUNELETTE_SESSION_MORE 2
/* service/session.h:7: selections one replay capture may hold. */
#define LUNELETTE_SESSION_REPLAY_TOKENS 16
/* service/native.c:632: the model's end-of-sequence id. */
#define LUNELETTE_SESSION_EOS 2

/* service/session.h:21-26: the receipt of the last materialize/restore, the
 * same fields in the same order. */
typedef struct {
    unsigned reused, full_attempted, full_committed, suffix_attempted, suffix_committed;
    unsigned pending_attempted, pending_committed, prefill_calls, append_calls, decode_calls;
    unsigned decode_attempted, decode_committed, logit_restores;
    unsigned recompute_attempted, recompute_committed;
} lunelette_session_work;

/* service/native.c:462-464 and service/session.h:53: 0 legacy (rebuild unless
 * the request appends exactly the pending non-EOS token), 1 reuse on (extend
 * the committed prefix, restore checkpoints), 2 off (recompute from the
 * start at every generation boundary and restore). */
typedef enum {
    LUNELETTE_SESSION_REUSE_LEGACY = 0,
    LUNELETTE_SESSION_REUSE_ON = 1,
    LUNELETTE_SESSION_REUSE_OFF = 2
} lunelette_session_reuse;

/* service/native.c:455-458, 503-507: context 256 or 4352, block 256 or 128,
 * block 256 when the context is 256. replay_path non-NULL selects the
 * controlled-replay evaluation mode: the file is created exclusively (an
 * existing file fails) and receives the LNRPLY1 header at open. */
typedef struct {
    size_t context, block;
    lunelette_session_reuse prefix_reuse;
    const char *replay_path;
} lunelette_session_options;

typedef struct lunelette_session lunelette_session;

/* service/native.c:431-560 without argv parsing, tokenizer or hashing:
 * admits the options, creates the replay file, loads the checkpoint with
 * lunelette_metal_create_configured(model, runtime, {context, block}) and
 * requires the reported strategy to be the requested one (no fallback).
 * NULL on failure, with a diagnostic in error; nothing stays open. */
lunelette_session *lunelette_session_open(const char *model,
    const lunelette_metal_options *runtime, const lunelette_session_options *options,
    char *error, size_t capacity);

/* Additive: the same admission over a context the caller already created
 * (a synthetic model, for instance) with the options in created. The
 * runtime's limits must equal {context, block} and its strategy
 * created->strategy. Ownership of runtime passes to the session on every
 * path: it is destroyed on failure. */
lunelette_session *lunelette_session_adopt(lunelette_metal *runtime,
    const lunelette_metal_options *created, const lunelette_session_options *options,
    char *error, size_t capacity);

/* service/native.c:107-117. NULL is allowed. */
void lunelette_session_destroy(lunelette_session *session);

/* service/native.c:161-255: bring the committed sequence to tokens[0..length)
 * by at most one runtime block per call (prefill for the first block,
 * decode for exactly the pending token, append otherwise). */
int lunelette_session_materialize(lunelette_session *session, const unsigned *tokens,
    unsigned length);
/* service/native.c:257-264: the same, reporting the committed length. */
int lunelette_session_materialize_step(lunelette_session *session, const unsigned *tokens,
    unsigned length, unsigned *cursor);

/* service/native.c:367-411: greedy selection over the current logits; the
 * token becomes pending until a materialize commits it. */
int lunelette_session_next(lunelette_session *session);
/* service/native.c:336-365, 413-416: replay mode only. Captures the record and
 * publishes the forced token (1000..131071 or EOS 2) instead of the greedy one. */
int lunelette_session_replay_next(lunelette_session *session, unsigned forced);

/* service/native.c:266-292 and 294-327. */
int lunelette_session_save(lunelette_session *session);
int lunelette_session_restore(lunelette_session *session);

/* service/native.c:78-82 (boundary), 84-89 (receipt), 65-76 (release the
 * checkpoint and stale logits, no model work) and 91-105 (empty sequence). */
void lunelette_session_begin(lunelette_session *session);
void lunelette_session_take_work(lunelette_session *session, lunelette_session_work *work);
void lunelette_session_invalidate(lunelette_session *session);
void lunelette_session_reset(lunelette_session *session);

/* Additive accessors: committed length, capacities, policy, the last
 * diagnostic ("" when none), the borrowed current logits (NULL when stale)
 * and the info object (service/native.c:562-616, its runtime fields). */
unsigned lunelette_session_length(const lunelette_session *session);
unsigned lunelette_session_context_capacity(const lunelette_session *session);
unsigned lunelette_session_block_capacity(const lunelette_session *session);
unsigned lunelette_session_prefix_reuse(const lunelette_session *session);
const char *lunelette_session_error(const lunelette_session *session);
const float *lunelette_session_logits(const lunelette_session *session);
const char *lunelette_session_info(const lunelette_session *session);

#ifdef __cplusplus
}
#endif

#endif
