/* Tokenizer and detokenizer of byte-level BPE vocabularies (the reference's cuda/text/,
 * declared in cuda/text/text.cuh): the vocabulary built from the arrays of a model file,
 * text cut into pre-tokens by the family's split pattern, each pre-token merged by pair
 * rank on the device, and token ids turned back into bytes. */
#ifndef AOTX_TEXT_H
#define AOTX_TEXT_H

#ifdef __cplusplus
extern "C" {
#endif

#define AOTX_TEXT_NONE        0xFFFFFFFFu   /* no token / no rank: cuda/text/text.cuh:14 */
#define AOTX_TEXT_CHUNK_BYTES 4096u         /* longest pre-token merged whole: text.cuh:24 */
#define AOTX_TEXT_TYPE_CONTROL 3            /* token types of the model file: text.cuh:41-43 */
#define AOTX_TEXT_TYPE_USER    4

/* Split patterns: the rows of cuda/text/families.h:10-14, in that order. */
#define AOTX_TEXT_PATTERN_QWEN2  0u
#define AOTX_TEXT_PATTERN_LLAMA3 1u
#define AOTX_TEXT_PATTERN_GPT2   2u
#define AOTX_TEXT_PATTERN_QWEN35 3u

/* The arrays of a model file that make a vocabulary (cuda/text/text.cuh:128-137). Host
 * memory: tokenizer.ggml.tokens as one byte run with tokens + 1 offsets, the merges
 * ("left right") the same way, tokenizer.ggml.token_type (may be null), and the family
 * row that aotx_text_family_find gives for tokenizer.ggml.pre. */
typedef struct aotx_text_source {
    const unsigned char *token_bytes;
    const unsigned long long *token_at;
    unsigned long long tokens;
    const unsigned char *merge_bytes;
    const unsigned long long *merge_at;
    unsigned long long merges;
    const int *token_type;
    unsigned int family;
} aotx_text_source;

/* The device memory of a built vocabulary (cuda/text/text.cuh:146-150). */
typedef struct aotx_text_store {
    void *block[8];
    unsigned int blocks;
    unsigned long long bytes;
} aotx_text_store;

/* The row of the family table that a tokenizer.ggml.pre value names; 0 when a row has
 * that name (cuda/text/text.cuh:142, vocab_host.cu:53-63). */
int aotx_text_family_find(const char *name, unsigned long long length, unsigned int *row);

/* Build the vocabulary on the device (cuda/text/text.cuh:154, vocab_host.cu:65-175): a
 * token table by string, a pair table by (left, right) with the merge rank and the merged
 * token, the token of each single byte, and the control bits. Returns 0 when the tables
 * are ready; 1 for a bad source (no tokens, a byte with no token, or an unknown family).
 * The vocabulary stays current until aotx_text_vocab_release. */
int aotx_text_vocab_build(const aotx_text_source *source, aotx_text_store *store);
void aotx_text_vocab_release(aotx_text_store *store);

/* Build the vocabulary from an open model file (include/aotx_modelfile.h):
 * tokenizer.ggml.tokens, .merges, .token_type and .pre (family row 0 when absent), as the
 * reference's load reads them into aotx_text_source. Returns 1 when the file has no
 * tokens, names an unknown family, or the build refuses the arrays. */
struct aotx_modelfile;
int aotx_text_vocab_file(const struct aotx_modelfile *file, aotx_text_store *store);

/* Counts of the last build: tokens, merges taken, merges refused (a side or the merged
 * string is not a token), control tokens. */
int aotx_text_vocab_report(unsigned int report[4]);

/* Encode `texts` byte runs (device: bytes, at[texts + 1] offsets) with the current
 * vocabulary: the tokens of text t go to ids + 3 * at[t] (ids holds 3 * at[texts]: a
 * byte that starts no UTF-8 character is read as U+FFFD, three bytes, as
 * cuda/text/text.cuh:367-374 cleans text, and a text never has more tokens than cleaned
 * bytes) and their count to count[t]. The pipeline of cuda/text/pretok.cu:393 and
 * bpe.cu:44-223: one thread per text cuts the pre-tokens (a pre-token longer than
 * AOTX_TEXT_CHUNK_BYTES is cut at a character boundary and the rest is matched again),
 * one wave per pre-token merges it (the lowest pair rank first, the leftmost of equal
 * ranks; with the family's whole rule a pre-token that is a token stays whole). Tokens
 * of the control and user types are whole matches found first, the longest at the
 * leftmost place (cuda/text/pretok.cu:339-372, :404-431); the pattern reads no text across
 * them. Returns 1 with no vocabulary or a bad argument; synchronous. */
int aotx_text_encode(const unsigned char *bytes, const unsigned long long *at, unsigned int texts,
                     unsigned int *ids, unsigned int *count, void *stream);

/* Turn tokens back into bytes (cuda/text/detok.cu:10-44): text t is tokens
 * ids[at[t] .. at[t + 1]) (device), its bytes go to bytes + t * limit and their count to
 * length[t] (cut at limit). Byte-level code points give their byte; other code points
 * keep their UTF-8; control tokens and ids past the vocabulary give nothing. Returns 1
 * with no vocabulary or a bad argument; asynchronous on the stream. */
int aotx_text_detok(const unsigned int *ids, const unsigned long long *at, unsigned int texts,
                    unsigned char *bytes, unsigned int limit, unsigned int *length, void *stream);

#ifdef __cplusplus
}
#endif

#endif
