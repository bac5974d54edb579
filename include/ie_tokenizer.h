/*
 * ie_tokenizer.h — GPT-2 byte-level BPE tokenizer for text prompts (host
 * code, no GPU).  C ABI over BPETokenizer (ie_bpe_tokenizer.h), which mirrors
 * the reference's BPETokenizer (include/tokenizer.h:7-25,
 * src/tokenizer.cpp:55-217): vocab.json and merges.txt read from the model
 * directory (python/export_gpt2.py:174-179 copies them there), words split at
 * whitespace, each after the first prefixed with the space byte, greedy
 * lowest-rank merges, unknown pieces dropped.  Functions return ie_status
 * codes (ie_amd.h); the message is in ie_last_error().
 */
#ifndef IE_TOKENIZER_H
#define IE_TOKENIZER_H

#include <stddef.h>

#include "ie_amd.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ie_tokenizer ie_tokenizer;

/* BPETokenizer(model_dir) (src/tokenizer.cpp:55-131): IE_ERR_INVALID when
 * vocab.json or merges.txt is missing or vocab.json is not a JSON object of
 * string keys and integer ids (the reference prints a message and exits). */
int ie_tokenizer_create(ie_tokenizer** out, const char* model_dir);
int ie_tokenizer_destroy(ie_tokenizer* t);
/* encode(text) (src/tokenizer.cpp:169-189) of len bytes of text: writes the
 * first min(*n_ids, cap) ids to ids and the full count to *n_ids, so a call
 * with cap 0 (ids may be NULL) sizes the buffer. */
int ie_tokenizer_encode(const ie_tokenizer* t, const char* text, size_t len, int* ids, size_t cap,
                        size_t* n_ids);
/* decode(token_ids) (src/tokenizer.cpp:191-217): the bytes of the ids in
 * order (ids outside [0, vocab_size) contribute nothing); writes the first
 * min(*n_bytes, cap) bytes to out and the full length to *n_bytes (no NUL). */
int ie_tokenizer_decode(const ie_tokenizer* t, const int* ids, size_t n, char* out, size_t cap,
                        size_t* n_bytes);
/* vocab_size() and eos_token() (include/tokenizer.h:15-16): 50257 and 50256,
 * as the reference's fixed-size id table; -1 for a NULL handle. */
int ie_tokenizer_vocab_size(const ie_tokenizer* t);
int ie_tokenizer_eos_token(const ie_tokenizer* t);

#ifdef __cplusplus
}
#endif

#endif /* IE_TOKENIZER_H */
