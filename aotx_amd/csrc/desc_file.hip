/* A model descriptor from a GGUF file, and the placement of its tensors (host only).
 *
 * Reference: cuda/model/desc_file_host.cu:18-298 (shape keys, the nearest layer kind,
 * bindings), cuda/model/kinds.h:70-121 (keys per kind), cuda/model/kinds_data.h:100-150
 * (tensor names per kind), cuda/model/rope_families.h:16-37 (pair rule per architecture),
 * cuda/model/desc.cu:30-90 (what binding a tensor writes into the descriptor).
 *
 * Kinds this build runs: attention with per-head Q/K norm (qwen3), attention without it
 * (llama), and routed experts without it (the Mixtral layout, whose GGUF names the llama
 * architecture). A layer holding tensors outside its kind, and any tensor whose type or
 * dimensions differ from what the descriptor implies, is refused here, before a kernel
 * could read past a tensor.
 */
#include "aotx_internal.h"
#include "modelfile.h"

#include <limits.h>
#include <string.h>

#include <string>
#include <vector>

namespace {

struct KindTensor {
    const char *name;
    unsigned int slot;
};

const KindTensor kind_attention[] = {
    {"attn_norm.weight", AOTX_SLOT_ATTN_NORM}, {"attn_q.weight", AOTX_SLOT_ATTN_Q},
    {"attn_k.weight", AOTX_SLOT_ATTN_K}, {"attn_v.weight", AOTX_SLOT_ATTN_V},
    {"attn_output.weight", AOTX_SLOT_ATTN_O}, {"attn_q_norm.weight", AOTX_ATTENTION_Q_NORM},
    {"attn_k_norm.weight", AOTX_ATTENTION_K_NORM}, {"ffn_norm.weight", AOTX_SLOT_FFN_NORM},
    {"ffn_gate.weight", AOTX_SLOT_FFN_GATE}, {"ffn_up.weight", AOTX_SLOT_FFN_UP},
    {"ffn_down.weight", AOTX_SLOT_FFN_DOWN}};
const KindTensor kind_no_qk_norm[] = {
    {"attn_norm.weight", AOTX_SLOT_ATTN_NORM}, {"attn_q.weight", AOTX_SLOT_ATTN_Q},
    {"attn_k.weight", AOTX_SLOT_ATTN_K}, {"attn_v.weight", AOTX_SLOT_ATTN_V},
    {"attn_output.weight", AOTX_SLOT_ATTN_O}, {"ffn_norm.weight", AOTX_SLOT_FFN_NORM},
    {"ffn_gate.weight", AOTX_SLOT_FFN_GATE}, {"ffn_up.weight", AOTX_SLOT_FFN_UP},
    {"ffn_down.weight", AOTX_SLOT_FFN_DOWN}};
const KindTensor kind_experts[] = {
    {"attn_norm.weight", AOTX_SLOT_ATTN_NORM}, {"attn_q.weight", AOTX_SLOT_ATTN_Q},
    {"attn_k.weight", AOTX_SLOT_ATTN_K}, {"attn_v.weight", AOTX_SLOT_ATTN_V},
    {"attn_output.weight", AOTX_SLOT_ATTN_O}, {"ffn_norm.weight", AOTX_SLOT_FFN_NORM},
    {"ffn_gate_exps.weight", AOTX_SLOT_FFN_GATE}, {"ffn_up_exps.weight", AOTX_SLOT_FFN_UP},
    {"ffn_down_exps.weight", AOTX_SLOT_FFN_DOWN}, {"ffn_gate_inp.weight", AOTX_EXPERT_ROUTER}};

struct Kind {
    unsigned int id;
    const KindTensor *tensor;
    unsigned int tensors;
};

const Kind kinds[] = {
    {AOTX_LAYER_KIND_ATTENTION, kind_attention, sizeof kind_attention / sizeof kind_attention[0]},
    {AOTX_LAYER_KIND_ATTENTION_NO_QK_NORM, kind_no_qk_norm,
     sizeof kind_no_qk_norm / sizeof kind_no_qk_norm[0]},
    {AOTX_LAYER_KIND_FFN_EXPERTS, kind_experts, sizeof kind_experts / sizeof kind_experts[0]}};

const Kind *kind_of(unsigned int id)
{
    for (const Kind &k : kinds)
        if (k.id == id) return &k;
    return nullptr;
}

/* The whole-model names (names.h:17-19), by descriptor slot order. */
const char *const whole_name[AOTX_DESC_WHOLE] = {"token_embd.weight", "output_norm.weight",
                                                 "output.weight", "cls.output.weight",
                                                 "rope_freqs.weight"};

bool has(const aotx_modelfile *f, const std::string &name)
{
    aotx_tensor_info info;
    return aotx_modelfile_find(f, name.c_str(), &info) == 0;
}

std::string layer_name(unsigned int layer, const char *tail)
{
    return "blk." + std::to_string(layer) + "." + tail;
}

/* The nearest kind of a layer (desc_file_host.cu:78-124): the kind's tensors the file
 * lacks plus the file's tensors of other kinds the kind lacks; the first least wins. */
unsigned int select_kind(const aotx_modelfile *f, unsigned int layer)
{
    unsigned int best = 0xffu, least = UINT_MAX;
    for (const Kind &cand : kinds) {
        unsigned int diff = 0;
        for (unsigned int i = 0; i < cand.tensors; ++i)
            if (!has(f, layer_name(layer, cand.tensor[i].name))) diff += 1;
        std::vector<std::string> counted;
        for (const Kind &other : kinds)
            for (unsigned int i = 0; i < other.tensors; ++i) {
                const char *n = other.tensor[i].name;
                bool in_cand = false;
                for (unsigned int j = 0; j < cand.tensors; ++j)
                    if (strcmp(cand.tensor[j].name, n) == 0) in_cand = true;
                bool seen = false;
                for (const std::string &c : counted)
                    if (c == n) seen = true;
                if (in_cand || seen) continue;
                counted.push_back(n);
                if (has(f, layer_name(layer, n))) diff += 1;
            }
        if (diff < least) {
            least = diff;
            best = cand.id;
        }
    }
    return best;
}

int fail(char *reason, size_t size, const char *fmt, const char *a = "", unsigned int b = 0u,
         unsigned int c = 0u)
{
    snprintf(reason, size, fmt, a, b, c);
    return 1;
}

/* rope_families.h:16-37 */
bool rope_pairs_of(const std::string &arch, unsigned int *pairs)
{
    static const struct {
        const char *name;
        unsigned int pairs;
    } table[] = {{"llama", AOTX_ROPE_PAIRS_ADJACENT}, {"olmo", AOTX_ROPE_PAIRS_ADJACENT},
                 {"qwen2", AOTX_ROPE_PAIRS_SPLIT},    {"qwen3", AOTX_ROPE_PAIRS_SPLIT},
                 {"qwen3moe", AOTX_ROPE_PAIRS_SPLIT}, {"olmoe", AOTX_ROPE_PAIRS_SPLIT},
                 {"qwen35", AOTX_ROPE_PAIRS_SPLIT}};
    for (const auto &row : table)
        if (arch == row.name) {
            *pairs = row.pairs;
            return true;
        }
    return false;
}

/* A u32 key "<arch>.<tail>": 0, or 1 with a reason (absent only when optional). */
int key_u32(const aotx_modelfile *f, const std::string &arch, const char *tail, unsigned int *v,
            bool needed, bool *present, char *reason, size_t size)
{
    const std::string key = arch + "." + tail;
    uint32_t got = 0;
    const int st = aotx_modelfile_u32(f, key.c_str(), &got);
    if (present != nullptr) *present = st == 0;
    if (st == 1 && !needed) return 0;
    if (st != 0)
        return fail(reason, size, st == 1 ? "the model file does not hold %s"
                                          : "the model key %s has an incompatible type",
                    key.c_str());
    *v = got;
    return 0;
}

int key_f32(const aotx_modelfile *f, const std::string &arch, const char *tail, float *v,
            char *reason, size_t size)
{
    const std::string key = arch + "." + tail;
    if (aotx_modelfile_f32(f, key.c_str(), v) != 0)
        return fail(reason, size, "the model file does not hold %s", key.c_str());
    return 0;
}

/* The type and dimensions a bound tensor must have (GGUF dims: fastest first). */
struct Want {
    unsigned int types;              /* bit mask of allowed types */
    uint64_t dims[3];
    unsigned int dim_count;
};

bool shape_ok(const aotx_tensor_info &t, const Want &w)
{
    if (((w.types >> t.type) & 1u) == 0u) return false;
    /* trailing dimensions of 1 may be left out by the writer */
    for (unsigned int d = 0; d < AOTX_TENSOR_DIMS; ++d) {
        const uint64_t want = d < w.dim_count ? w.dims[d] : 1u;
        const uint64_t got = d < t.dim_count ? t.dims[d] : 1u;
        if (want != got) return false;
    }
    return true;
}

Want want_of(const aotx_model_desc *d, unsigned int slot)
{
    const uint64_t h = d->hidden, hd = d->head_dim, wide = (uint64_t)d->heads * hd,
                   narrow = (uint64_t)d->kv_heads * hd, f = d->ffn, e = d->expert_count;
    const unsigned int q8 = 1u << AOTX_TENSOR_Q8_0, f32 = 1u << AOTX_TENSOR_F32;
    const unsigned int embd = q8 | (1u << AOTX_TENSOR_F16) | f32;
    if (slot < AOTX_DESC_WHOLE) {
        switch (slot) {
        case 0: return {embd, {h, d->vocab, 1}, 2};
        case 1: return {f32, {h, 1, 1}, 1};
        case 2: return {q8, {h, d->vocab, 1}, 2};
        case 3: return {0u, {0, 0, 0}, 0};            /* classifier heads are not run */
        default: return {f32, {hd / 2u, 1, 1}, 1};
        }
    }
    const unsigned int s = (slot - AOTX_DESC_WHOLE) % AOTX_LAYER_TENSOR_SLOTS;
    const unsigned int layer = (slot - AOTX_DESC_WHOLE) / AOTX_LAYER_TENSOR_SLOTS;
    const bool experts = d->kind[layer] == AOTX_LAYER_KIND_FFN_EXPERTS;
    switch (s) {
    case AOTX_SLOT_ATTN_NORM: case AOTX_SLOT_FFN_NORM: return {f32, {h, 1, 1}, 1};
    case AOTX_SLOT_ATTN_Q: return {q8, {h, wide, 1}, 2};
    case AOTX_SLOT_ATTN_K: case AOTX_SLOT_ATTN_V: return {q8, {h, narrow, 1}, 2};
    case AOTX_SLOT_ATTN_O: return {q8, {wide, h, 1}, 2};
    case AOTX_ATTENTION_Q_NORM: case AOTX_ATTENTION_K_NORM: return {f32, {hd, 1, 1}, 1};
    case AOTX_SLOT_FFN_GATE: case AOTX_SLOT_FFN_UP:
        return experts ? Want{q8, {h, f, e}, 3} : Want{q8, {h, f, 1}, 2};
    case AOTX_SLOT_FFN_DOWN:
        return experts ? Want{q8, {f, h, e}, 3} : Want{q8, {f, h, 1}, 2};
    case AOTX_EXPERT_ROUTER: return {f32, {h, e, 1}, 2};
    default: return {0u, {0, 0, 0}, 0};
    }
}

} // namespace

extern "C" int aotx_model_desc_file(const aotx_modelfile *file, unsigned int role,
                                    aotx_model_desc *desc, aotx_model_binding *binding,
                                    unsigned int capacity, unsigned int *count, char *reason,
                                    size_t reason_size)
{
    if (file == nullptr || desc == nullptr || binding == nullptr || count == nullptr
        || reason == nullptr || reason_size == 0u || role >= AOTX_MODEL_ROLES)
        return 1;
    reason[0] = '\0';
    *count = 0u;
    memset(desc, 0, sizeof *desc);
    memset(desc->kind, 0xff, sizeof desc->kind);
    for (unsigned int l = 0; l < AOTX_MODEL_MAX_LAYERS; ++l)
        for (unsigned int s = 0; s < AOTX_LAYER_TENSOR_SLOTS; ++s) desc->layer[l].offset[s] = AOTX_MODEL_ABSENT;
    desc->role = role;
    desc->tied_output = 1u;
    desc->token_embd = desc->output_norm = desc->output = AOTX_MODEL_ABSENT;
    desc->cls_output = desc->rope_freqs = AOTX_MODEL_ABSENT;
    if (role != AOTX_MODEL_LANGUAGE && role != AOTX_MODEL_LANGUAGE_Q4 && role != AOTX_MODEL_LANGUAGE_AUDIO)
        return fail(reason, reason_size, "%sthe role %u is not a language role", "", role);

    /* ---- shape (desc_file_host.cu:126-228) ---- */
    const char *a = nullptr;
    size_t alen = 0;
    if (aotx_modelfile_string(file, "general.architecture", &a, &alen) != 0 || alen == 0u
        || alen >= 64u)
        return fail(reason, reason_size, "the model file does not name an architecture");
    const std::string arch(a, alen);
    if (key_u32(file, arch, "block_count", &desc->layers, true, nullptr, reason, reason_size)
        || key_u32(file, arch, "embedding_length", &desc->hidden, true, nullptr, reason, reason_size)
        || key_u32(file, arch, "context_length", &desc->context, true, nullptr, reason, reason_size)
        || key_u32(file, arch, "pooling_type", &desc->pooling, false, nullptr, reason, reason_size))
        return 1;
    if (desc->layers == 0u || desc->layers > AOTX_MODEL_MAX_LAYERS)
        return fail(reason, reason_size, "%sthe layer count %u is outside the bounds", "", desc->layers);
    if (!rope_pairs_of(arch, &desc->rope_pairs))
        return fail(reason, reason_size, "the architecture %s has no rotary pair rule", arch.c_str());
    if (desc->pooling != 0u)
        return fail(reason, reason_size, "%sa language model asks for the pooling %u", "", desc->pooling);
    bool selected[3] = {false, false, false};
    for (unsigned int l = 0; l < desc->layers; ++l) {
        desc->kind[l] = (unsigned char)select_kind(file, l);
        selected[desc->kind[l]] = true;
    }
    /* keys of the selected kinds (kinds.h:70-121) */
    bool hd_present = false;
    if (key_u32(file, arch, "feed_forward_length", &desc->ffn, true, nullptr, reason, reason_size)
        || key_u32(file, arch, "attention.head_count", &desc->heads, true, nullptr, reason, reason_size)
        || key_u32(file, arch, "attention.head_count_kv", &desc->kv_heads, true, nullptr, reason, reason_size)
        || key_u32(file, arch, "attention.key_length", &desc->head_dim,
                   selected[AOTX_LAYER_KIND_ATTENTION], &hd_present, reason, reason_size)
        || key_f32(file, arch, "rope.freq_base", &desc->rope_theta, reason, reason_size)
        || key_f32(file, arch, "attention.layer_norm_rms_epsilon", &desc->rms_eps, reason, reason_size))
        return 1;
    if (selected[AOTX_LAYER_KIND_FFN_EXPERTS]
        && (key_u32(file, arch, "expert_count", &desc->expert_count, true, nullptr, reason, reason_size)
            || key_u32(file, arch, "expert_used_count", &desc->expert_used_count, true, nullptr,
                       reason, reason_size)))
        return 1;
    if (desc->heads == 0u || desc->kv_heads == 0u || desc->heads % desc->kv_heads != 0u)
        return fail(reason, reason_size, "the head count is outside the bounds");
    if (!hd_present && desc->hidden % desc->heads == 0u) desc->head_dim = desc->hidden / desc->heads;
    if (desc->head_dim != 64u && desc->head_dim != 128u)
        return fail(reason, reason_size, "%sthe head width %u is not one this build runs (64, 128)", "",
                    desc->head_dim);
    if (desc->expert_count > AOTX_LAYER_EXPERTS_MAX || desc->expert_used_count > desc->expert_count)
        return fail(reason, reason_size, "the expert counts are outside the bounds");
    desc->weight_type = AOTX_WEIGHT_Q8_0;

    /* ---- bindings (desc_file_host.cu:230-266) ---- */
    unsigned int needed = AOTX_DESC_WHOLE;
    for (unsigned int l = 0; l < desc->layers; ++l) needed += kind_of(desc->kind[l])->tensors;
    if (capacity < needed) return fail(reason, reason_size, "the tensor binding list is too small");
    unsigned int n = 0;
    for (unsigned int i = 0; i < AOTX_DESC_WHOLE; ++i, ++n) {
        snprintf(binding[n].name, sizeof binding[n].name, "%s", whole_name[i]);
        binding[n].slot = i;
        binding[n].needed = i < 2u ? 1u : 0u;
    }
    for (unsigned int l = 0; l < desc->layers; ++l) {
        const Kind *k = kind_of(desc->kind[l]);
        for (unsigned int i = 0; i < k->tensors; ++i, ++n) {
            const std::string name = layer_name(l, k->tensor[i].name);
            if (name.size() >= sizeof binding[n].name)
                return fail(reason, reason_size, "a tensor name does not fit the binding list");
            snprintf(binding[n].name, sizeof binding[n].name, "%s", name.c_str());
            binding[n].slot = AOTX_DESC_WHOLE + l * AOTX_LAYER_TENSOR_SLOTS + k->tensor[i].slot;
            binding[n].needed = 1u;
        }
    }
    *count = n;
    unsigned int missing = 0, first = 0;
    for (unsigned int i = 0; i < n; ++i)
        if (binding[i].needed && !has(file, binding[i].name)) {
            if (missing == 0u) first = i;
            missing += 1u;
        }
    if (missing != 0u)
        return fail(reason, reason_size, "the model has no tensor %s, and %u more are absent",
                    binding[first].name, missing - 1u);

    /* ---- every layer tensor of the file belongs to its layer's kind ---- */
    const uint64_t tensors = aotx_modelfile_tensor_count(file);
    for (uint64_t t = 0; t < tensors; ++t) {
        aotx_tensor_info info;
        if (aotx_modelfile_tensor(file, t, &info) != 0) continue;
        unsigned int l = 0;
        int used = 0;
        if (sscanf(info.name, "blk.%u.%n", &l, &used) != 1 || used == 0) continue;
        if (l >= desc->layers)
            return fail(reason, reason_size, "the tensor %s is past the layer count", info.name);
        bool known = false;
        for (unsigned int i = 0; i < n; ++i)
            if (strcmp(binding[i].name, info.name) == 0) known = true;
        if (!known)
            return fail(reason, reason_size, "the tensor %s is outside its layer's kind", info.name);
    }

    /* ---- the vocabulary, then every bound tensor's type and dimensions ---- */
    aotx_tensor_info emb;
    aotx_modelfile_find(file, whole_name[0], &emb);
    if (emb.dim_count < 2u || emb.dims[1] == 0u || emb.dims[1] > 0x7fffffffu)
        return fail(reason, reason_size, "the token embedding has no row count");
    desc->vocab = (unsigned int)emb.dims[1];
    for (unsigned int i = 0; i < n; ++i) {
        aotx_tensor_info info;
        if (aotx_modelfile_find(file, binding[i].name, &info) != 0) continue;
        if (!shape_ok(info, want_of(desc, binding[i].slot)))
            return fail(reason, reason_size, "the tensor %s has a type or shape this model does not take",
                        binding[i].name);
    }
    return 0;
}

static unsigned long long place_align(unsigned long long v)
{
    return (v + 255ull) / 256ull * 256ull;
}

extern "C" unsigned long long aotx_model_place_bytes(const aotx_modelfile *file,
                                                     const aotx_model_binding *binding,
                                                     unsigned int count)
{
    if (file == nullptr || binding == nullptr) return 0ull;
    unsigned long long at = 0ull;
    for (unsigned int i = 0; i < count; ++i) {
        aotx_tensor_info info;
        if (aotx_modelfile_find(file, binding[i].name, &info) != 0) continue;
        at = place_align(at) + info.bytes;
    }
    return place_align(at);
}

unsigned long long aotx_mem_weights_bytes(void);

extern "C" int aotx_model_place(const aotx_modelfile *file, aotx_model_desc *desc,
                                const aotx_model_binding *binding, unsigned int count,
                                char *reason, size_t reason_size)
{
    if (file == nullptr || desc == nullptr || binding == nullptr || reason == nullptr
        || reason_size == 0u)
        return 1;
    reason[0] = '\0';
    const unsigned long long base = aotx_mem_weights_base();
    const unsigned long long need = aotx_model_place_bytes(file, binding, count);
    if (base == 0ull || aotx_mem_weights_bytes() < need)
        return fail(reason, reason_size, "the weights region is absent or smaller than the file's tensors");
    const size_t piece = 64u << 20;
    std::vector<unsigned char> buf;
    unsigned long long at = 0ull;
    for (unsigned int i = 0; i < count; ++i) {
        aotx_tensor_info info;
        const unsigned int slot = binding[i].slot;
        unsigned long long *dst;
        if (slot < AOTX_DESC_WHOLE) {
            unsigned long long *whole[AOTX_DESC_WHOLE] = {&desc->token_embd, &desc->output_norm,
                                                          &desc->output, &desc->cls_output,
                                                          &desc->rope_freqs};
            dst = whole[slot];
        } else {
            const unsigned int s = slot - AOTX_DESC_WHOLE;
            dst = &desc->layer[s / AOTX_LAYER_TENSOR_SLOTS].offset[s % AOTX_LAYER_TENSOR_SLOTS];
        }
        if (aotx_modelfile_find(file, binding[i].name, &info) != 0) {
            *dst = AOTX_MODEL_ABSENT;
            if (binding[i].needed) return fail(reason, reason_size, "the model has no tensor %s", binding[i].name);
            continue;
        }
        at = place_align(at);
        if (buf.empty()) buf.resize(piece);
        for (unsigned long long done = 0; done < info.bytes;) {
            const size_t take = (size_t)((info.bytes - done) < piece ? (info.bytes - done) : piece);
            if (aotx_modelfile_read(file, info.offset + done, take, buf.data()) != 0)
                return fail(reason, reason_size, "the tensor %s did not read", binding[i].name);
            AOTX_CHECK(hipMemcpy((void *)(base + at + done), buf.data(), take, hipMemcpyHostToDevice));
            done += take;
        }
        *dst = at;
        /* what the bind writes besides the offset (desc.cu:66-88) */
        if (slot == 0u) desc->embd_type = info.type;
        if (slot == 2u) desc->tied_output = 0u;
        if (slot >= AOTX_DESC_WHOLE) {
            const unsigned int s = slot - AOTX_DESC_WHOLE;
            desc->layer_type[s / AOTX_LAYER_TENSOR_SLOTS][s % AOTX_LAYER_TENSOR_SLOTS] = (unsigned char)info.type;
        }
        if (slot == AOTX_DESC_WHOLE + AOTX_SLOT_ATTN_Q) desc->weight_type = info.type;
        at += info.bytes;
    }
    return 0;
}
