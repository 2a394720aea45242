/* GGUF model files and the model descriptor built from one (C ABI, host only).
 *
 * Replaces the reference's reader disk/modelfile/modelfile.h:110-160 (format constants
 * :22-95, tensor info :97-111, string arrays :113-119) and its descriptor builder
 * cuda/model/forward.cuh:290-302 (aotx_model_binding, aotx_model_desc_file, from
 * cuda/model/desc_file_host.cu:268-298). Placement (aotx_model_place) has no single
 * counterpart: the reference streams tensors into the weights region from its load queue
 * and binds offsets by name on the device (cuda/model/desc.cu:30-90); here one host call
 * does both for one file.
 *
 * Codes: 0 ran; 1 the file cannot be read (or a key / tensor / index is absent); 2 the
 * format is wrong (or a value has another type). Not thread-safe per file.
 */
#ifndef AOTX_MODELFILE_H
#define AOTX_MODELFILE_H

#include <stddef.h>
#include <stdint.h>

#include "aotx_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* modelfile.h:22-24 */
#define AOTX_GGUF_MAGIC        0x46554747u   /* "GGUF" read as a little-endian u32 */
#define AOTX_GGUF_VERSION      3u
#define AOTX_GGUF_ALIGN        32u

/* modelfile.h:27-39: metadata value types */
#define AOTX_GGUF_U8           0u
#define AOTX_GGUF_I8           1u
#define AOTX_GGUF_U16          2u
#define AOTX_GGUF_I16          3u
#define AOTX_GGUF_U32          4u
#define AOTX_GGUF_I32          5u
#define AOTX_GGUF_F32          6u
#define AOTX_GGUF_BOOL         7u
#define AOTX_GGUF_STRING       8u
#define AOTX_GGUF_ARRAY        9u
#define AOTX_GGUF_U64          10u
#define AOTX_GGUF_I64          11u
#define AOTX_GGUF_F64          12u

/* modelfile.h:43-54: tensor types whose bytes stream (others open but do not stream) */
#define AOTX_TENSOR_F32        0u
#define AOTX_TENSOR_F16        1u
#define AOTX_TENSOR_Q4_0       2u
#define AOTX_TENSOR_Q4_1       3u
#define AOTX_TENSOR_Q5_0       6u
#define AOTX_TENSOR_Q5_1       7u
#define AOTX_TENSOR_Q8_0       8u
#define AOTX_TENSOR_Q2_K       10u
#define AOTX_TENSOR_Q3_K       11u
#define AOTX_TENSOR_Q4_K       12u
#define AOTX_TENSOR_Q5_K       13u
#define AOTX_TENSOR_Q6_K       14u

/* gguf.h:12-24: bounds of what a file may make the reader hold */
#define AOTX_GGUF_HEAD_LIMIT   (256u * 1024u * 1024u)
#define AOTX_GGUF_MEMORY_LIMIT (512u * 1024u * 1024u)
#define AOTX_GGUF_PAIR_LEAST   12u
#define AOTX_GGUF_TENSOR_LEAST 24u
#define AOTX_GGUF_KEY_BYTES    256u

#define AOTX_TENSOR_NAME_BYTES 128u
#define AOTX_TENSOR_DIMS       4u

/* modelfile.h:97-104 */
typedef struct aotx_tensor_info {
    char     name[AOTX_TENSOR_NAME_BYTES];
    uint32_t dim_count;
    uint32_t type;
    uint64_t dims[AOTX_TENSOR_DIMS];
    uint64_t offset;            /* from the start of the tensor bytes */
    uint64_t bytes;             /* from the dimensions and the type; 0 for a type that does
                                   not stream */
} aotx_tensor_info;

/* modelfile.h:113-119 */
typedef struct aotx_string_array {
    uint64_t count;
    const uint8_t *bytes;
    const uint64_t *offsets;    /* count + 1 entries; string i is [offsets[i], offsets[i+1]) */
} aotx_string_array;

typedef struct aotx_modelfile aotx_modelfile;

/* modelfile.h:123-128: open and check the header, metadata and tensor table */
int aotx_modelfile_open(const char *path, aotx_modelfile **file);
void aotx_modelfile_close(aotx_modelfile *file);
/* modelfile.h:140-141 */
uint64_t aotx_modelfile_file_bytes(const aotx_modelfile *file);
uint64_t aotx_modelfile_header_bytes(const aotx_modelfile *file);
/* modelfile.h:143-157: metadata by key (0; 1 absent; 2 another type or out of range) */
int aotx_modelfile_u32(const aotx_modelfile *file, const char *key, uint32_t *value);
int aotx_modelfile_u64(const aotx_modelfile *file, const char *key, uint64_t *value);
int aotx_modelfile_f32(const aotx_modelfile *file, const char *key, float *value);
int aotx_modelfile_string(const aotx_modelfile *file, const char *key, const char **value,
                          size_t *length);
int aotx_modelfile_strings(const aotx_modelfile *file, const char *key,
                           aotx_string_array *array);
int aotx_modelfile_i32s(const aotx_modelfile *file, const char *key, const int32_t **values,
                        uint64_t *count);
int aotx_modelfile_f32s(const aotx_modelfile *file, const char *key, const float **values,
                        uint64_t *count);
int aotx_modelfile_bools(const aotx_modelfile *file, const char *key, const uint8_t **values,
                         uint64_t *count);
/* modelfile.h:153-160: the tensor table and tensor bytes (offset from the tensor bytes) */
uint64_t aotx_modelfile_tensor_count(const aotx_modelfile *file);
int aotx_modelfile_tensor(const aotx_modelfile *file, uint64_t index, aotx_tensor_info *info);
int aotx_modelfile_find(const aotx_modelfile *file, const char *name, aotx_tensor_info *info);
uint64_t aotx_modelfile_data_bytes(const aotx_modelfile *file);
int aotx_modelfile_read(const aotx_modelfile *file, uint64_t offset, uint64_t bytes,
                        void *buffer);

/* cuda/model/names.h:12-19 and forward.cuh:290-294 */
#define AOTX_DESC_WHOLE        5u            /* token_embd, output_norm, output, cls.output, rope_freqs */
#define AOTX_DESC_BUFFER       48u
#define AOTX_DESC_MAX_BINDINGS (AOTX_DESC_WHOLE + AOTX_MODEL_MAX_LAYERS * AOTX_LAYER_TENSOR_SLOTS)

typedef struct aotx_model_binding {
    char name[AOTX_DESC_BUFFER];
    unsigned int slot;          /* < AOTX_DESC_WHOLE: a whole-model tensor; else
                                   AOTX_DESC_WHOLE + layer * AOTX_LAYER_TENSOR_SLOTS + slot */
    unsigned int needed;
} aotx_model_binding;

/* forward.cuh:296-302 (desc_file_host.cu:268-298): the descriptor of one file for a role
 * (shape from the metadata, each layer's kind by the tensors it holds) and its bindings.
 * Tensor offsets are left absent; 1 with a diagnostic in reason when the file cannot make
 * a runnable descriptor. Uses no GPU. */
int aotx_model_desc_file(const aotx_modelfile *file, unsigned int role, aotx_model_desc *desc,
                         aotx_model_binding *binding, unsigned int capacity,
                         unsigned int *count, char *reason, size_t reason_size);

/* Bytes of the weights region that aotx_model_place needs for these bindings. */
unsigned long long aotx_model_place_bytes(const aotx_modelfile *file,
                                          const aotx_model_binding *binding,
                                          unsigned int count);
/* Copy every bound tensor of the file into the weights region (aotx_mem_weights_set;
 * 256-byte aligned, in binding order) and fill the descriptor as the reference's bind does
 * (desc.cu:30-90): offsets, each layer tensor's type, the embedding type and vocabulary,
 * and the head (a file without output.weight ties the head to the embedding). 0, or 1
 * with a diagnostic in reason. */
int aotx_model_place(const aotx_modelfile *file, aotx_model_desc *desc,
                     const aotx_model_binding *binding, unsigned int count,
                     char *reason, size_t reason_size);

#ifdef __cplusplus
}
#endif

#endif
