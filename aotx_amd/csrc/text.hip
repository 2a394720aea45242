/* Byte-level BPE tokenizer and detokenizer (the reference's cuda/text/).
 *
 * The vocabulary is built on the host from the model file's arrays and copied to the
 * device once: a token table by string (FNV-1a, open addressing), a pair table by (left,
 * right) that holds the merge rank and the merged token (so the merge step never joins
 * strings), the token of each single byte, and the control bits.
 *
 * Encoding is three launches:
 *   - pre-tokens: one thread per text runs the family's split pattern, a state machine
 *     that takes the first alternative matching at a position (cuda/text/pretok.cu:1-45);
 *   - merge: one 64-lane workgroup per pre-token (a work list the pre-token pass appends
 *     to) holds its symbols in LDS as a linked list
 *     with the rank of each symbol's pair; each round a wave minimum over (rank, position)
 *     picks the pair to merge (the lowest rank, the leftmost of equal ranks), and only
 *     the two pairs next to it are looked up again;
 *   - gather: one wave per text copies its pre-tokens' tokens in order.
 * Detokenizing is one wave per text: token lengths, a wave prefix sum, then the bytes.
 */
#include "aotx_internal.h"
#include "unicode_classes.h"
#include "../../include/aotx_text.h"
#include "../../include/aotx_modelfile.h"

#include <stdlib.h>
#include <string.h>

#include <string>
#include <unordered_map>
#include <vector>

/* ---- character classes and UTF-8 -------------------------------------------------------- */

static __device__ int uc_in(const unsigned int *r, unsigned int n, unsigned int cp)
{
    unsigned int lo = 0u, hi = n;            /* ranges [2i, 2i + 1], sorted */
    while (lo < hi) {
        const unsigned int mid = (lo + hi) >> 1;
        if (cp < r[2u * mid]) hi = mid;
        else if (cp > r[2u * mid + 1u]) lo = mid + 1u;
        else return 1;
    }
    return 0;
}
static __device__ __forceinline__ int is_letter(unsigned int p)
{
    if (p < 0x80u) return (p >= 'A' && p <= 'Z') || (p >= 'a' && p <= 'z');
    return uc_in(aotx_uc_letter, AOTX_UC_LETTER_RANGES, p);
}
static __device__ __forceinline__ int is_number(unsigned int p)
{
    if (p < 0x80u) return p >= '0' && p <= '9';
    return uc_in(aotx_uc_number, AOTX_UC_NUMBER_RANGES, p);
}
static __device__ __forceinline__ int is_space(unsigned int p)
{
    if (p < 0x80u) return p == 0x20u || (p >= 0x09u && p <= 0x0Du);
    return uc_in(aotx_uc_space, AOTX_UC_SPACE_RANGES, p);
}
static __device__ __forceinline__ int is_mark(unsigned int p)
{
    return p >= 0x80u && uc_in(aotx_uc_mark, AOTX_UC_MARK_RANGES, p);
}

/* The code point at `at` and its byte count; a byte run that is not UTF-8 reads as
 * U+FFFD of one byte. */
static __device__ unsigned int utf8_at(const unsigned char *b, unsigned int end, unsigned int at,
                                       unsigned int *point)
{
    const unsigned int c = b[at];
    unsigned int need, cp, min;
    if (c < 0x80u) { *point = c; return 1u; }
    if ((c & 0xE0u) == 0xC0u) { need = 1u; cp = c & 0x1Fu; min = 0x80u; }
    else if ((c & 0xF0u) == 0xE0u) { need = 2u; cp = c & 0x0Fu; min = 0x800u; }
    else if ((c & 0xF8u) == 0xF0u) { need = 3u; cp = c & 0x07u; min = 0x10000u; }
    else { *point = 0xFFFDu; return 1u; }
    if (at + need >= end) { *point = 0xFFFDu; return 1u; }     /* cut off by the end */
    for (unsigned int i = 1u; i <= need; ++i) {
        const unsigned int d = b[at + i];
        if ((d & 0xC0u) != 0x80u) { *point = 0xFFFDu; return 1u; }
        cp = (cp << 6) | (d & 0x3Fu);
    }
    if (cp < min || cp > 0x10FFFFu || (cp >= 0xD800u && cp <= 0xDFFFu)) { *point = 0xFFFDu; return 1u; }
    *point = cp;
    return need + 1u;
}

/* The byte-level alphabet: each byte stands as one code point that is printable UTF-8
 * (the GPT-2 byte map; cuda/text/text.cuh:256-290). */
static __host__ __device__ __forceinline__ unsigned int byte_point(unsigned int b)
{
    if ((b >= 0x21u && b <= 0x7Eu) || (b >= 0xA1u && b <= 0xACu) || (b >= 0xAEu && b <= 0xFFu)) return b;
    if (b <= 0x20u) return 0x100u + b;
    if (b <= 0xA0u) return 0x100u + 33u + (b - 0x7Fu);
    return 0x100u + 67u;                                   /* 0xAD */
}
static __device__ __forceinline__ unsigned int point_byte(unsigned int p)
{
    if ((p >= 0x21u && p <= 0x7Eu) || (p >= 0xA1u && p <= 0xACu) || (p >= 0xAEu && p <= 0xFFu)) return p;
    if (p < 0x100u || p > 0x143u) return 0x100u;
    const unsigned int a = p - 0x100u;
    if (a <= 0x20u) return a;
    if (a <= 66u) return 0x7Fu + (a - 33u);
    return 0xADu;
}
static __host__ __device__ __forceinline__ unsigned int utf8_put(unsigned int p, unsigned char *o)
{
    if (p < 0x80u) { o[0] = (unsigned char)p; return 1u; }
    if (p < 0x800u) { o[0] = (unsigned char)(0xC0u | (p >> 6)); o[1] = (unsigned char)(0x80u | (p & 0x3Fu)); return 2u; }
    if (p < 0x10000u) {
        o[0] = (unsigned char)(0xE0u | (p >> 12)); o[1] = (unsigned char)(0x80u | ((p >> 6) & 0x3Fu));
        o[2] = (unsigned char)(0x80u | (p & 0x3Fu)); return 3u;
    }
    o[0] = (unsigned char)(0xF0u | (p >> 18)); o[1] = (unsigned char)(0x80u | ((p >> 12) & 0x3Fu));
    o[2] = (unsigned char)(0x80u | ((p >> 6) & 0x3Fu)); o[3] = (unsigned char)(0x80u | (p & 0x3Fu));
    return 4u;
}

static __host__ __device__ __forceinline__ unsigned long long fnv_step(unsigned long long h, unsigned int byte)
{
    return (h ^ (unsigned long long)byte) * 1099511628211ull;
}
#define FNV_BASIS 14695981039346656037ull
static __host__ __device__ __forceinline__ unsigned long long pair_mix(unsigned long long k)
{
    k ^= k >> 33; k *= 0xFF51AFD7ED558CCDull; k ^= k >> 33; k *= 0xC4CEB9FE1A85EC53ull; k ^= k >> 33;
    return k;
}

/* ---- the vocabulary ------------------------------------------------------------------- */

struct aotx_text_vocab {
    const unsigned char *token_bytes;
    const unsigned long long *token_at;
    unsigned int tokens;
    unsigned int slots;                 /* power of two */
    const unsigned int *slot;           /* token of each slot, or AOTX_TEXT_NONE */
    unsigned int pairs;                 /* power of two */
    const unsigned long long *pair_key; /* left << 32 | right, or all ones */
    const unsigned int *pair_rank;
    const unsigned int *pair_result;
    const unsigned int *control;        /* one bit per token */
    const unsigned int *special;        /* tokens of the control and user types */
    unsigned int specials;
    unsigned long long first[4];        /* bits of the first bytes of the specials */
    unsigned int pattern;
    unsigned int whole;
    unsigned int byte_token[256];
};

static aotx_text_vocab g_vocab;
static int g_ready = 0;
static unsigned int g_report[4];

static __device__ __forceinline__ unsigned int find_pair(const aotx_text_vocab &v, unsigned int l,
                                                         unsigned int r, unsigned int *result)
{
    if (l == AOTX_TEXT_NONE || r == AOTX_TEXT_NONE) return AOTX_TEXT_NONE;
    const unsigned long long key = ((unsigned long long)l << 32) | r;
    const unsigned int mask = v.pairs - 1u;
    unsigned int at = (unsigned int)pair_mix(key) & mask;
    for (unsigned int i = 0; i <= mask; ++i) {
        const unsigned long long got = v.pair_key[at];
        if (got == ~0ull) return AOTX_TEXT_NONE;
        if (got == key) { *result = v.pair_result[at]; return v.pair_rank[at]; }
        at = (at + 1u) & mask;
    }
    return AOTX_TEXT_NONE;
}

/* The token whose string is the byte-level form of bytes [0, n), or AOTX_TEXT_NONE. */
static __device__ unsigned int find_bytes(const aotx_text_vocab &v, const unsigned char *b, unsigned int n)
{
    unsigned long long h = FNV_BASIS;
    unsigned int len = 0u;
    for (unsigned int i = 0; i < n; ++i) {
        unsigned char u[4];
        const unsigned int k = utf8_put(byte_point(b[i]), u);
        for (unsigned int j = 0; j < k; ++j) h = fnv_step(h, u[j]);
        len += k;
    }
    const unsigned int mask = v.slots - 1u;
    unsigned int at = (unsigned int)h & mask;
    for (unsigned int step = 0; step <= mask; ++step) {
        const unsigned int t = v.slot[at];
        if (t == AOTX_TEXT_NONE) return AOTX_TEXT_NONE;
        const unsigned long long f = v.token_at[t];
        if (v.token_at[t + 1u] - f == len) {
            const unsigned char *s = v.token_bytes + f;
            unsigned int pos = 0u;
            bool same = true;
            for (unsigned int i = 0; i < n && same; ++i) {
                unsigned char u[4];
                const unsigned int k = utf8_put(byte_point(b[i]), u);
                for (unsigned int j = 0; j < k; ++j) same = same && s[pos + j] == u[j];
                pos += k;
            }
            if (same) return t;
        }
        at = (at + 1u) & mask;
    }
    return AOTX_TEXT_NONE;
}

/* ---- pre-tokens (cuda/text/pretok.cu:1-45 states the alternatives) -------------------- */

/* 's 't 're 've 'm 'll 'd at `at`, small letters (or any case); bytes of the match or 0 */
static __device__ unsigned int contraction(const unsigned char *b, unsigned int at, unsigned int end,
                                           int any_case)
{
    if (b[at] != '\'' || at + 1u >= end) return 0u;
    unsigned int c1 = b[at + 1u], c2 = at + 2u < end ? b[at + 2u] : 0u;
    if (any_case) {
        if (c1 >= 'A' && c1 <= 'Z') c1 += 32u;
        if (c2 >= 'A' && c2 <= 'Z') c2 += 32u;
    }
    if (c1 == 's' || c1 == 't' || c1 == 'm' || c1 == 'd') return 2u;
    if ((c1 == 'r' && c2 == 'e') || (c1 == 'v' && c2 == 'e') || (c1 == 'l' && c2 == 'l')) return 3u;
    return 0u;
}
static __device__ unsigned int letter_run(const unsigned char *b, unsigned int end, unsigned int at, int marks)
{
    while (at < end) {
        unsigned int p;
        const unsigned int k = utf8_at(b, end, at, &p);
        if (!(is_letter(p) || (marks && is_mark(p)))) break;
        at += k;
    }
    return at;
}
static __device__ unsigned int number_run(const unsigned char *b, unsigned int end, unsigned int at,
                                          unsigned int most)
{
    for (unsigned int n = 0u; at < end && (most == 0u || n < most); ++n) {
        unsigned int p;
        const unsigned int k = utf8_at(b, end, at, &p);
        if (!is_number(p)) break;
        at += k;
    }
    return at;
}
/* characters that are not space, letter or number (nor marks, when marks are letters) */
static __device__ unsigned int other_run(const unsigned char *b, unsigned int end, unsigned int at, int marks)
{
    while (at < end) {
        unsigned int p;
        const unsigned int k = utf8_at(b, end, at, &p);
        if (is_space(p) || is_letter(p) || is_number(p) || (marks && is_mark(p))) break;
        at += k;
    }
    return at;
}
/* the space alternatives at a space character: with the newline rule, \s*[\r\n]+ first;
 * then \s+(?!\S) (the run gives back its last character when a non-space follows); \s+ */
static __device__ unsigned int spaces(const unsigned char *b, unsigned int end, unsigned int at,
                                      unsigned int span, int newline_rule)
{
    unsigned int stop = at, last = at, newline = 0u;
    bool found = false;
    while (stop < end) {
        unsigned int p;
        const unsigned int k = utf8_at(b, end, stop, &p);
        if (!is_space(p)) break;
        if (p == '\r' || p == '\n') { newline = stop; found = true; }
        last = stop;
        stop += k;
    }
    if (stop == at) return span;
    if (newline_rule && found) return newline + 1u - at;
    if (stop == end) return stop - at;
    if (last > at) return last - at;
    return stop - at;
}
static __device__ unsigned int match(unsigned int pattern, const unsigned char *b, unsigned int at,
                                     unsigned int end)
{
    unsigned int first;
    const unsigned int span = utf8_at(b, end, at, &first);
    if (pattern == AOTX_TEXT_PATTERN_GPT2) {
        const unsigned int c = contraction(b, at, end, 0);
        if (c != 0u) return c;
        const unsigned int from = first == ' ' ? at + 1u : at;
        unsigned int walk = letter_run(b, end, from, 0);
        if (walk == from) walk = number_run(b, end, from, 0u);
        if (walk == from) walk = other_run(b, end, from, 0);
        if (walk > from) return walk - at;
        return spaces(b, end, at, span, 0);
    }
    const int marks = pattern == AOTX_TEXT_PATTERN_QWEN35;
    const unsigned int most = pattern == AOTX_TEXT_PATTERN_LLAMA3 ? 3u : 1u;
    const unsigned int c = contraction(b, at, end, 1);
    if (c != 0u) return c;
    {
        unsigned int from = at;
        if (first != '\r' && first != '\n' && !is_letter(first) && !is_number(first)
            && !(marks && is_mark(first)))
            from = at + span;
        const unsigned int walk = letter_run(b, end, from, marks);
        if (walk > from) return walk - at;
    }
    if (is_number(first)) return number_run(b, end, at, most) - at;
    {
        const unsigned int from = first == ' ' ? at + 1u : at;
        unsigned int walk = other_run(b, end, from, marks);
        if (walk > from) {
            while (walk < end && (b[walk] == '\r' || b[walk] == '\n')) walk += 1u;
            return walk - at;
        }
    }
    return spaces(b, end, at, span, 1);
}

/* one thread per text: the text with every byte that does not start a UTF-8 character
 * (and the bytes of a cut or malformed one) written as U+FFFD, EF BF BD (cuda/text/
 * text.cuh:367-374); text t goes to out + 3 at[t], its length to clean_len[t] */
__global__ void aotx_text_clean_kernel(const unsigned char *bytes, const unsigned long long *at,
                                       unsigned int texts, unsigned char *out,
                                       unsigned long long *at3, unsigned int *clean_len)
{
    const unsigned int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t > texts) return;
    at3[t] = 3ull * at[t];
    if (t == texts) return;
    const unsigned char *b = bytes + at[t];
    const unsigned int end = (unsigned int)(at[t + 1u] - at[t]);
    unsigned char *o = out + 3ull * at[t];
    unsigned int w = 0u;
    for (unsigned int pos = 0u; pos < end;) {
        unsigned int p;
        const unsigned int k = utf8_at(b, end, pos, &p);
        if (p == 0xFFFDu && k == 1u) {        /* no character starts here */
            o[w] = 0xEFu; o[w + 1u] = 0xBFu; o[w + 2u] = 0xBDu;
            w += 3u;
        } else {
            for (unsigned int i = 0u; i < k; ++i) o[w + i] = b[pos + i];
            w += k;
        }
        pos += k;
    }
    clean_len[t] = w;
}

/* The longest special token whose bytes start at `at` (cuda/text/pretok.cu:339-372): its
 * length, 0 for none. */
static __device__ unsigned int special_at(const aotx_text_vocab &v, const unsigned char *b,
                                          unsigned int at, unsigned int end, unsigned int *token)
{
    const unsigned int c = b[at];
    if (((v.first[c >> 6] >> (c & 63u)) & 1ull) == 0ull) return 0u;
    unsigned int best = 0u;
    for (unsigned int i = 0u; i < v.specials; ++i) {
        const unsigned int id = v.special[i];
        const unsigned long long f = v.token_at[id];
        const unsigned int n = (unsigned int)(v.token_at[id + 1u] - f);
        if (n <= best || at + n > end) continue;
        unsigned int k = 0u;
        while (k < n && v.token_bytes[f + k] == b[at + k]) k += 1u;
        if (k == n) { best = n; *token = id; }
    }
    return best;
}

/* one thread per text: pre-token p of text t is (start[at[t] + p], len[at[t] + p]), and
 * tok[at[t] + p] its token when it is a special token (else AOTX_TEXT_NONE). A special
 * token is a whole match and the pattern reads no text across it. */
__global__ void aotx_text_pretok_kernel(aotx_text_vocab v, const unsigned char *bytes,
                                        const unsigned long long *at, const unsigned int *clean_len,
                                        unsigned int texts, unsigned int *start, unsigned int *len,
                                        unsigned int *tok, unsigned int *pieces, unsigned int *work,
                                        unsigned int *works)
{
    const unsigned int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= texts) return;
    const unsigned long long base = at[t];
    const unsigned char *b = bytes + base;
    const unsigned int text_end = clean_len[t];
    unsigned int pos = 0u, n = 0u;
    while (pos < text_end) {
        unsigned int stop = pos, special = 0u, id = AOTX_TEXT_NONE;
        while (stop < text_end && v.specials != 0u) {
            special = special_at(v, b, stop, text_end, &id);
            if (special != 0u) break;
            stop += 1u;
        }
        if (v.specials == 0u) stop = text_end;
        const unsigned int end = stop;
        while (pos < end) {
        unsigned int m = match(v.pattern, b, pos, end);
        if (m == 0u) m = 1u;
        if (m > AOTX_TEXT_CHUNK_BYTES) {          /* cut at a character boundary */
            unsigned int cut = 0u;
            while (cut < end - pos) {
                unsigned int p;
                const unsigned int k = utf8_at(b, end, pos + cut, &p);
                if (cut + k > AOTX_TEXT_CHUNK_BYTES) break;
                cut += k;
            }
            m = cut;
        }
        start[base + n] = pos;
        len[base + n] = m;
        tok[base + n] = AOTX_TEXT_NONE;
        n += 1u;
        pos += m;
        }
        if (special != 0u) {
            start[base + n] = stop;
            len[base + n] = special;
            tok[base + n] = id;
            n += 1u;
            pos = stop + special;
        }
    }
    pieces[t] = n;
    /* the merge step takes one workgroup per pre-token of the batch, from this list */
    const unsigned int first = atomicAdd(works, n);
    for (unsigned int i = 0u; i < n; ++i) work[first + i] = (unsigned int)(base + i);
}

/* ---- merge: one 64-lane workgroup per pre-token slot ----------------------------------- */

#define TX_N AOTX_TEXT_CHUNK_BYTES

__global__ __launch_bounds__(64) void aotx_text_merge_kernel(aotx_text_vocab v, const unsigned char *bytes,
                                                             const unsigned long long *at, unsigned int texts,
                                                             const unsigned int *start, const unsigned int *len,
                                                             const unsigned int *ptok,
                                                             const unsigned int *pieces, const unsigned int *work,
                                                             unsigned int *out, unsigned int *out_count)
{
    __shared__ unsigned int tok[TX_N], rank[TX_N], res[TX_N];
    __shared__ unsigned short nxt[TX_N], prv[TX_N];
    const unsigned int lane = threadIdx.x;
    const unsigned long long s = work[blockIdx.x];
    /* the text of slot s: at[t] <= s < at[t + 1] */
    unsigned int lo = 0u, hi = texts;
    while (hi - lo > 1u) {
        const unsigned int mid = (lo + hi) >> 1;
        if (at[mid] <= s) lo = mid; else hi = mid;
    }
    const unsigned int t = lo;
    if (s - at[t] >= pieces[t]) return;
    const unsigned char *b = bytes + at[t] + start[s];
    const unsigned int n = len[s];
    /* a pre-token's tokens (never more than its bytes) go where its bytes are */
    unsigned int *dst = out + at[t] + start[s];
    if (ptok[s] != AOTX_TEXT_NONE) {
        if (lane == 0u) { dst[0] = ptok[s]; out_count[s] = 1u; }
        return;
    }
    if (v.whole) {
        const unsigned int w = lane == 0u ? find_bytes(v, b, n) : 0u;
        const unsigned int whole = __shfl(w, 0, 64);
        if (whole != AOTX_TEXT_NONE) {
            if (lane == 0u) { dst[0] = whole; out_count[s] = 1u; }
            return;
        }
    }
    for (unsigned int i = lane; i < n; i += 64u) {
        tok[i] = v.byte_token[b[i]];
        nxt[i] = (unsigned short)(i + 1u);
        prv[i] = (unsigned short)(i == 0u ? 0xFFFFu : i - 1u);
    }
    __syncthreads();
    for (unsigned int i = lane; i < n; i += 64u) {
        unsigned int r = 0u;
        rank[i] = i + 1u < n ? find_pair(v, tok[i], tok[i + 1u], &r) : AOTX_TEXT_NONE;
        res[i] = r;
    }
    __syncthreads();
    for (;;) {
        unsigned long long best = ~0ull;
        for (unsigned int i = lane; i < n; i += 64u) {
            const unsigned long long k = ((unsigned long long)rank[i] << 32) | i;
            best = k < best ? k : best;
        }
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) {
            const unsigned long long o = __shfl_xor(best, d, 64);
            best = o < best ? o : best;
        }
        if ((unsigned int)(best >> 32) == AOTX_TEXT_NONE) break;
        if (lane == 0u) {
            const unsigned int i = (unsigned int)best, j = nxt[i];
            tok[i] = res[i];
            const unsigned int k = nxt[j];
            nxt[i] = (unsigned short)k;
            if (k < n) prv[k] = (unsigned short)i;
            rank[j] = AOTX_TEXT_NONE;
            unsigned int r = 0u;
            rank[i] = k < n ? find_pair(v, tok[i], tok[k], &r) : AOTX_TEXT_NONE;
            res[i] = r;
            const unsigned int p = prv[i];
            if (p != 0xFFFFu) {
                unsigned int r2 = 0u;
                rank[p] = find_pair(v, tok[p], tok[i], &r2);
                res[p] = r2;
            }
        }
        __syncthreads();
    }
    if (lane == 0u) {
        unsigned int c = 0u;
        for (unsigned int i = 0u; i < n; i = nxt[i]) dst[c++] = tok[i];
        out_count[s] = c;
    }
}

/* one wave per text: its pre-tokens' tokens, in order, to ids + at[t] */
__global__ __launch_bounds__(64) void aotx_text_gather_kernel(const unsigned long long *at,
                                                              const unsigned int *start,
                                                              const unsigned int *pieces,
                                                              const unsigned int *piece_tokens,
                                                              const unsigned int *piece_count,
                                                              unsigned int *ids, unsigned int *count)
{
    const unsigned int t = blockIdx.x, lane = threadIdx.x;
    const unsigned long long base = at[t];
    unsigned int w = 0u;
    for (unsigned int p = 0u; p < pieces[t]; ++p) {
        const unsigned int c = piece_count[base + p];
        const unsigned int *src = piece_tokens + base + start[base + p];
        for (unsigned int i = lane; i < c; i += 64u) ids[base + w + i] = src[i];
        w += c;
    }
    if (lane == 0u) count[t] = w;
}

/* ---- detokenize ------------------------------------------------------------------------ */

static __device__ unsigned int detok_token(const aotx_text_vocab &v, unsigned int id, unsigned char *o,
                                           unsigned int room)
{
    if (id >= v.tokens || ((v.control[id >> 5] >> (id & 31u)) & 1u)) return 0u;
    const unsigned char *s = v.token_bytes + v.token_at[id];
    const unsigned int n = (unsigned int)(v.token_at[id + 1u] - v.token_at[id]);
    unsigned int w = 0u;
    for (unsigned int i = 0u; i < n;) {
        unsigned int p;
        const unsigned int k = utf8_at(s, n, i, &p);
        const unsigned int byte = point_byte(p);
        if (byte < 0x100u) {
            if (o != nullptr && w < room) o[w] = (unsigned char)byte;
            w += 1u;
        } else {
            for (unsigned int j = 0u; j < k; ++j) {
                if (o != nullptr && w < room) o[w] = s[i + j];
                w += 1u;
            }
        }
        i += k;
    }
    return w;
}

__global__ __launch_bounds__(64) void aotx_text_detok_kernel(aotx_text_vocab v, const unsigned int *ids,
                                                             const unsigned long long *at, unsigned char *bytes,
                                                             unsigned int limit, unsigned int *length)
{
    const unsigned int t = blockIdx.x, lane = threadIdx.x;
    const unsigned long long a0 = at[t], a1 = at[t + 1u];
    unsigned char *dst = bytes + (unsigned long long)t * limit;
    unsigned int w = 0u;
    for (unsigned long long c = a0; c < a1; c += 64u) {
        const unsigned long long i = c + lane;
        const unsigned int mine = i < a1 ? detok_token(v, ids[i], nullptr, 0u) : 0u;
        unsigned int incl = mine;
#pragma unroll
        for (unsigned int d = 1u; d < 64u; d <<= 1) {
            const unsigned int o = __shfl_up(incl, d, 64);
            if (lane >= d) incl += o;
        }
        const unsigned int from = w + incl - mine;
        if (i < a1 && from < limit) detok_token(v, ids[i], dst + from, limit - from);
        w += __shfl(incl, 63, 64);
    }
    if (lane == 0u) length[t] = w < limit ? w : limit;
}

/* ---- host -------------------------------------------------------------------------------- */

struct aotx_text_family { const char *name; unsigned int pattern, whole; };
/* cuda/text/families.h:24-43: tokenizer.ggml.pre value, split pattern, whole rule */
static const aotx_text_family kFamilies[] = {
    {"qwen2", AOTX_TEXT_PATTERN_QWEN2, 0u}, {"deepseek-r1-qwen", AOTX_TEXT_PATTERN_QWEN2, 0u},
    {"kormo", AOTX_TEXT_PATTERN_QWEN2, 0u}, {"f2llmv2", AOTX_TEXT_PATTERN_QWEN2, 0u},
    {"llama3", AOTX_TEXT_PATTERN_LLAMA3, 1u}, {"llama-v3", AOTX_TEXT_PATTERN_LLAMA3, 1u},
    {"llama-bpe", AOTX_TEXT_PATTERN_LLAMA3, 1u}, {"falcon3", AOTX_TEXT_PATTERN_LLAMA3, 1u},
    {"falcon-h1", AOTX_TEXT_PATTERN_LLAMA3, 1u}, {"pixtral", AOTX_TEXT_PATTERN_LLAMA3, 1u},
    {"midm-2.0", AOTX_TEXT_PATTERN_LLAMA3, 1u}, {"lfm2", AOTX_TEXT_PATTERN_LLAMA3, 1u},
    {"jina-v5-nano", AOTX_TEXT_PATTERN_LLAMA3, 1u}, {"gpt-2", AOTX_TEXT_PATTERN_GPT2, 0u},
    {"mpt", AOTX_TEXT_PATTERN_GPT2, 0u}, {"olmo", AOTX_TEXT_PATTERN_GPT2, 0u},
    {"jais", AOTX_TEXT_PATTERN_GPT2, 0u}, {"trillion", AOTX_TEXT_PATTERN_GPT2, 0u},
    {"granite-docling", AOTX_TEXT_PATTERN_GPT2, 0u}, {"qwen35", AOTX_TEXT_PATTERN_QWEN35, 0u},
};
static const unsigned int kFamilyCount = sizeof kFamilies / sizeof kFamilies[0];

extern "C" int aotx_text_family_find(const char *name, unsigned long long length, unsigned int *row)
{
    if (name == nullptr || row == nullptr) return 1;
    for (unsigned int i = 0; i < kFamilyCount; ++i) {
        if (strlen(kFamilies[i].name) == length && memcmp(kFamilies[i].name, name, length) == 0) {
            *row = i;
            return 0;
        }
    }
    return 1;
}

static unsigned int pow2_at_least(unsigned long long n)
{
    unsigned int p = 16u;
    while (p < n) p <<= 1;
    return p;
}

template <class T>
static T *store_put(aotx_text_store *st, const T *src, size_t count)
{
    void *d = nullptr;
    const size_t bytes = count * sizeof(T) > 0 ? count * sizeof(T) : sizeof(T);
    AOTX_CHECK(hipMalloc(&d, bytes));
    if (count) AOTX_CHECK(hipMemcpy(d, src, count * sizeof(T), hipMemcpyHostToDevice));
    st->block[st->blocks++] = d;
    st->bytes += bytes;
    return (T *)d;
}

extern "C" void aotx_text_vocab_release(aotx_text_store *store)
{
    if (store == nullptr) return;
    for (unsigned int i = 0; i < store->blocks; ++i) AOTX_CHECK(hipFree(store->block[i]));
    store->blocks = 0u;
    store->bytes = 0ull;
    g_ready = 0;
}

extern "C" int aotx_text_vocab_build(const aotx_text_source *src, aotx_text_store *store)
{
    if (src == nullptr || store == nullptr || src->tokens == 0ull || src->tokens >= 0xFFFFFFFFull
        || src->token_bytes == nullptr || src->token_at == nullptr || src->family >= kFamilyCount
        || (src->merges != 0ull && (src->merge_bytes == nullptr || src->merge_at == nullptr)))
        return 1;
    const unsigned int n = (unsigned int)src->tokens;
    std::unordered_map<std::string, unsigned int> id;
    id.reserve(n * 2u);
    for (unsigned int t = 0; t < n; ++t) {
        std::string s((const char *)src->token_bytes + src->token_at[t], src->token_at[t + 1u] - src->token_at[t]);
        id.emplace(s, t);                                /* the lowest id of a repeated string */
    }
    /* the token table by string */
    const unsigned int slots = pow2_at_least(2ull * n);
    std::vector<unsigned int> slot(slots, AOTX_TEXT_NONE);
    for (unsigned int t = 0; t < n; ++t) {
        const unsigned long long f = src->token_at[t], e = src->token_at[t + 1u];
        std::string s((const char *)src->token_bytes + f, e - f);
        if (id[s] != t) continue;
        unsigned long long h = FNV_BASIS;
        for (unsigned long long i = f; i < e; ++i) h = fnv_step(h, src->token_bytes[i]);
        unsigned int at = (unsigned int)h & (slots - 1u);
        while (slot[at] != AOTX_TEXT_NONE) at = (at + 1u) & (slots - 1u);
        slot[at] = t;
    }
    /* the pair table: rank = merge index, result = the token of the joined string */
    const unsigned int pairs = pow2_at_least(2ull * (src->merges + 1ull));
    std::vector<unsigned long long> key(pairs, ~0ull);
    std::vector<unsigned int> rank(pairs, AOTX_TEXT_NONE), result(pairs, AOTX_TEXT_NONE);
    unsigned int taken = 0u, refused = 0u;
    for (unsigned long long m = 0; m < src->merges; ++m) {
        std::string line((const char *)src->merge_bytes + src->merge_at[m], src->merge_at[m + 1u] - src->merge_at[m]);
        const size_t sp = line.find(' ', 1);
        if (sp == std::string::npos) { refused += 1u; continue; }
        const std::string l = line.substr(0, sp), r = line.substr(sp + 1);
        auto il = id.find(l), ir = id.find(r), ij = id.find(l + r);
        if (il == id.end() || ir == id.end() || ij == id.end()) { refused += 1u; continue; }
        const unsigned long long k = ((unsigned long long)il->second << 32) | ir->second;
        unsigned int at = (unsigned int)pair_mix(k) & (pairs - 1u);
        bool seen = false;
        while (key[at] != ~0ull) {
            if (key[at] == k) { seen = true; break; }
            at = (at + 1u) & (pairs - 1u);
        }
        if (seen) { refused += 1u; continue; }              /* a repeated pair keeps its first rank */
        key[at] = k;
        rank[at] = (unsigned int)m;
        result[at] = ij->second;
        taken += 1u;
    }
    /* control bits and the single bytes */
    std::vector<unsigned int> control((n + 31u) / 32u, 0u);
    unsigned int controls = 0u;
    if (src->token_type != nullptr)
        for (unsigned int t = 0; t < n; ++t)
            if (src->token_type[t] == AOTX_TEXT_TYPE_CONTROL) { control[t >> 5] |= 1u << (t & 31u); controls += 1u; }
    aotx_text_vocab v;
    memset(&v, 0, sizeof v);
    std::vector<unsigned int> special;
    if (src->token_type != nullptr)
        for (unsigned int t = 0; t < n; ++t)
            if ((src->token_type[t] == AOTX_TEXT_TYPE_CONTROL || src->token_type[t] == AOTX_TEXT_TYPE_USER)
                && src->token_at[t + 1u] > src->token_at[t]) {
                special.push_back(t);
                const unsigned int c = src->token_bytes[src->token_at[t]];
                v.first[c >> 6] |= 1ull << (c & 63u);
            }
    for (unsigned int b = 0; b < 256u; ++b) {
        unsigned char u[4];
        const unsigned int k = utf8_put(byte_point(b), u);
        auto it = id.find(std::string((const char *)u, k));
        if (it == id.end()) return 1;
        v.byte_token[b] = it->second;
    }
    aotx_text_vocab_release(store);
    v.token_bytes = store_put(store, src->token_bytes, src->token_at[n]);
    v.token_at = store_put(store, src->token_at, (size_t)n + 1u);
    v.tokens = n;
    v.slots = slots;
    v.slot = store_put(store, slot.data(), slots);
    v.pairs = pairs;
    v.pair_key = store_put(store, key.data(), pairs);
    v.pair_rank = store_put(store, rank.data(), pairs);
    v.pair_result = store_put(store, result.data(), pairs);
    v.control = store_put(store, control.data(), control.size());
    v.special = store_put(store, special.data(), special.size());
    v.specials = (unsigned int)special.size();
    v.pattern = kFamilies[src->family].pattern;
    v.whole = kFamilies[src->family].whole;
    g_vocab = v;
    g_ready = 1;
    g_report[0] = n;
    g_report[1] = taken;
    g_report[2] = refused;
    g_report[3] = controls;
    return 0;
}

extern "C" int aotx_text_vocab_file(const aotx_modelfile *file, aotx_text_store *store)
{
    if (file == nullptr || store == nullptr) return 1;
    aotx_string_array tokens, merges;
    memset(&merges, 0, sizeof merges);
    if (aotx_modelfile_strings(file, "tokenizer.ggml.tokens", &tokens) != 0) return 1;
    if (aotx_modelfile_strings(file, "tokenizer.ggml.merges", &merges) != 0) merges.count = 0u;
    const int32_t *types = nullptr;
    uint64_t type_count = 0u;
    if (aotx_modelfile_i32s(file, "tokenizer.ggml.token_type", &types, &type_count) != 0
        || type_count != tokens.count)
        types = nullptr;
    const char *pre = nullptr;
    size_t pre_len = 0u;
    unsigned int family = 0u;                       /* row 0 when the file names none */
    if (aotx_modelfile_string(file, "tokenizer.ggml.pre", &pre, &pre_len) == 0
        && aotx_text_family_find(pre, pre_len, &family) != 0)
        return 1;
    aotx_text_source src;
    src.token_bytes = tokens.bytes;
    src.token_at = (const unsigned long long *)tokens.offsets;
    src.tokens = tokens.count;
    src.merge_bytes = merges.count ? merges.bytes : nullptr;
    src.merge_at = merges.count ? (const unsigned long long *)merges.offsets : nullptr;
    src.merges = merges.count;
    src.token_type = types;
    src.family = family;
    return aotx_text_vocab_build(&src, store);
}

extern "C" int aotx_text_vocab_report(unsigned int report[4])
{
    if (report == nullptr || !g_ready) return 1;
    memcpy(report, g_report, sizeof g_report);
    return 0;
}

extern "C" int aotx_text_encode(const unsigned char *bytes, const unsigned long long *at, unsigned int texts,
                                unsigned int *ids, unsigned int *count, void *stream)
{
    if (!g_ready || bytes == nullptr || at == nullptr || ids == nullptr || count == nullptr || texts == 0u)
        return 1;
    hipStream_t s = aotx_stream(stream);
    unsigned long long total = 0ull;
    AOTX_CHECK(hipMemcpyAsync(&total, at + texts, sizeof total, hipMemcpyDeviceToHost, s));
    AOTX_CHECK(hipStreamSynchronize(s));
    if (total == 0ull) {
        AOTX_CHECK(hipMemsetAsync(count, 0, texts * sizeof(unsigned int), s));
        AOTX_CHECK(hipStreamSynchronize(s));
        return 0;
    }
    unsigned int *start = nullptr, *len = nullptr, *pieces = nullptr, *ptok = nullptr, *pcount = nullptr,
                 *pspecial = nullptr, *clean_len = nullptr;
    unsigned char *clean = nullptr;
    unsigned long long *at3 = nullptr;
    const unsigned long long room = 3ull * total;       /* every byte may become U+FFFD */
    AOTX_CHECK(hipMallocAsync((void **)&clean, room, s));
    AOTX_CHECK(hipMallocAsync((void **)&at3, (texts + 1ull) * 8u, s));
    AOTX_CHECK(hipMallocAsync((void **)&clean_len, texts * 4u, s));
    AOTX_CHECK(hipMallocAsync((void **)&start, room * 4u, s));
    AOTX_CHECK(hipMallocAsync((void **)&len, room * 4u, s));
    AOTX_CHECK(hipMallocAsync((void **)&ptok, room * 4u, s));
    AOTX_CHECK(hipMallocAsync((void **)&pcount, room * 4u, s));
    AOTX_CHECK(hipMallocAsync((void **)&pspecial, room * 4u, s));
    AOTX_CHECK(hipMallocAsync((void **)&pieces, texts * 4u, s));
    unsigned int *work = nullptr, *works = nullptr;
    AOTX_CHECK(hipMallocAsync((void **)&work, room * 4u, s));
    AOTX_CHECK(hipMallocAsync((void **)&works, 4u, s));
    AOTX_CHECK(hipMemsetAsync(works, 0, 4u, s));
    hipLaunchKernelGGL(aotx_text_clean_kernel, dim3((texts + 64u) / 64u), dim3(64), 0, s, bytes, at, texts,
                       clean, at3, clean_len);
    AOTX_LAUNCH_CHECK();
    hipLaunchKernelGGL(aotx_text_pretok_kernel, dim3((texts + 63u) / 64u), dim3(64), 0, s, g_vocab, clean, at3,
                       clean_len, texts, start, len, pspecial, pieces, work, works);
    AOTX_LAUNCH_CHECK();
    unsigned int nwork = 0u;
    AOTX_CHECK(hipMemcpyAsync(&nwork, works, 4u, hipMemcpyDeviceToHost, s));
    AOTX_CHECK(hipStreamSynchronize(s));
    if (nwork > 0u) {
        hipLaunchKernelGGL(aotx_text_merge_kernel, dim3(nwork), dim3(64), 0, s, g_vocab, clean, at3, texts,
                           start, len, pspecial, pieces, work, ptok, pcount);
        AOTX_LAUNCH_CHECK();
    }
    hipLaunchKernelGGL(aotx_text_gather_kernel, dim3(texts), dim3(64), 0, s, at3, start, pieces, ptok, pcount,
                       ids, count);
    AOTX_LAUNCH_CHECK();
    void *tmp[] = {clean, at3, clean_len, start, len, ptok, pcount, pspecial, pieces, work, works};
    for (void *q : tmp) AOTX_CHECK(hipFreeAsync(q, s));
    AOTX_CHECK(hipStreamSynchronize(s));
    return 0;
}

extern "C" int aotx_text_detok(const unsigned int *ids, const unsigned long long *at, unsigned int texts,
                               unsigned char *bytes, unsigned int limit, unsigned int *length, void *stream)
{
    if (!g_ready || ids == nullptr || at == nullptr || bytes == nullptr || length == nullptr || texts == 0u)
        return 1;
    hipLaunchKernelGGL(aotx_text_detok_kernel, dim3(texts), dim3(64), 0, aotx_stream(stream), g_vocab, ids, at,
                       bytes, limit, length);
    AOTX_LAUNCH_CHECK();
    return 0;
}
