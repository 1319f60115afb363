/* Byte-level BPE tokenizer over the reference's exported files: replaces
 * toyinfer::Tokenizer and toyinfer::MergeRank (include/tokenizer.h:11-57;
 * src/tokenizer.cpp:22-381).  Host code: the prompt is tokenised once per
 * request and the ids are then copied to the device.
 *
 * Files in model_dir, as export.py writes them (export.py:49-135, 138-188):
 *   tokenizer.bin  u32 count, then per token id: u32 length, raw bytes;
 *   merges.bin     u32 count, then per merge rank: u32 left id, u32 right id,
 *                  u32 merged id;
 *   template_user.txt, template_system.txt (and *_thinking.txt): the chat
 *                  template with %s for the user (and system) text.
 * Integers are little-endian.  Ids from count to vocab_size - 1 (the padded
 * vocabulary) have empty text.
 *
 * Status codes are those of include/toyinfer_attn.h; TOYINFER_ERR_IO for a
 * missing or malformed file (where the reference throws). */
#ifndef TOYINFER_TOKENIZER_H_
#define TOYINFER_TOKENIZER_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct toyinfer_tokenizer toyinfer_tokenizer;

/* Loads the vocabulary, the merge table and the two templates of the
 * thinking or non-thinking mode (src/tokenizer.cpp:64-135).  A token count
 * above vocab_size is TOYINFER_ERR_IO, as the reference's check (:91-94). */
int toyinfer_tokenizer_create(const char* model_dir, uint32_t vocab_size, int thinking,
                              toyinfer_tokenizer** out);
void toyinfer_tokenizer_destroy(toyinfer_tokenizer* t);

/* Tokenizer::encode (src/tokenizer.cpp:169-325): text is split into special
 * tokens ("<...>" found whole in the vocabulary, the first '>' within the
 * longest token length) and single bytes; then adjacent pairs merge, the
 * lowest merge rank first and the leftmost among equal ranks, until no pair
 * in the merge table remains.  Writes min(count, cap) ids; *count is the
 * full number (TOYINFER_ERR_WORKSPACE when it exceeds cap).  A byte with no
 * single-byte token is TOYINFER_ERR_INVALID_ARGUMENT (the reference throws). */
int toyinfer_tokenizer_encode(toyinfer_tokenizer* t, const char* text, uint32_t* ids,
                              uint32_t cap, uint32_t* count);

/* Tokenizer::decode (src/tokenizer.cpp:327-333): the token's bytes
 * (NUL-terminated, owned by the tokenizer and valid until destroy), NULL for
 * an id at or above vocab_size.  *len (if not NULL) receives the byte length,
 * which counts embedded NUL bytes.  A tokenizer is read-only after create:
 * encode, decode and render_prompt may run on several threads at once. */
const char* toyinfer_tokenizer_decode(const toyinfer_tokenizer* t, uint32_t id, uint32_t* len);

/* Tokenizer::render_prompt (src/tokenizer.cpp:335-369): the system template
 * with (system_prompt, user_prompt) when both are given, else the user
 * template with user_prompt.  "%s" takes the next argument and "%%" is a
 * percent sign, as in the reference's snprintf; any other '%' sequence is
 * TOYINFER_ERR_INVALID_ARGUMENT (the template is never used as a format).
 * Writes at most cap bytes including the NUL; *len is the full length
 * without it (TOYINFER_ERR_WORKSPACE when it does not fit). */
int toyinfer_tokenizer_render_prompt(const toyinfer_tokenizer* t, const char* user_prompt,
                                     const char* system_prompt, char* buf, size_t cap,
                                     size_t* len);

/* Size of the loaded vocabulary (vocab_size) and the number of merges. */
uint32_t toyinfer_tokenizer_vocab_size(const toyinfer_tokenizer* t);
uint32_t toyinfer_tokenizer_num_merges(const toyinfer_tokenizer* t);

#ifdef __cplusplus
}
#endif

#endif /* TOYINFER_TOKENIZER_H_ */
