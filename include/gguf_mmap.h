/* gguf_mmap.h -- C ABI of the GGUF reader in libpurhie_qmv.so: the on-disk format that feeds the matvecs.
 *
 * Drop-in for the reference's src/gguf_mmap.h:15-121 (same names, argument meaning and return conventions), plus
 * what replaces its host-pinned weights on MI355X: the tensors copied once into HBM (gguf_hbm_bytes /
 * gguf_hbm_stage, in place of src/model_stage.h:1-38 and pin_model_memory, src/inference.cpp:274) and the
 * engine's bind_weight (src/inference.cpp:362-389) as gguf_bind_weight.
 *
 * Files are GGUF version 3, optionally split as <prefix>-00001-of-0000N.gguf (opened by the first). Unlike the
 * reference, every header, key, array and tensor extent is checked against the file size at open: a truncated
 * or inconsistent file is refused (NULL) instead of read out of bounds. */
#ifndef PURHIE_GGUF_MMAP_H
#define PURHIE_GGUF_MMAP_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct gguf_model gguf_model_t;

/* replaces src/gguf_mmap.h:15-17: open (NULL on any error) / close / a tensor's bytes by name */
gguf_model_t *gguf_mmap_open(const char *path);
void gguf_mmap_close(gguf_model_t *model);
const void *gguf_mmap_get_tensor(const gguf_model_t *model, const char *name, size_t *out_bytes);

/* replaces src/gguf_mmap.h:20-31: tensor introspection by index. ne has 4 entries, those past n_dims 0 (as the
 * reference's zero-filled table). Sizes: block_size / type_size from the GGML type table ((size_t)-1 for a type
 * it does not know), row_size = ceil(ne[0] / block) blocks rounded up to 32 bytes, nbytes = floor(elements /
 * block) blocks, nbytes_pad = nbytes. Out-of-range indices: "(null)", -1, NULL, 0 or (size_t)-1 as the
 * reference. */
int64_t gguf_n_tensors(const gguf_model_t *model);
const char *gguf_tensor_name(const gguf_model_t *model, int64_t idx);
int gguf_tensor_type(const gguf_model_t *model, int64_t idx);
int64_t *gguf_tensor_ne(const gguf_model_t *model, int64_t idx);
uint8_t gguf_tensor_dims(const gguf_model_t *model, int64_t idx);
size_t gguf_tensor_block_size(const gguf_model_t *model, int64_t idx);
size_t gguf_tensor_type_size(const gguf_model_t *model, int64_t idx);
size_t gguf_tensor_row_size(const gguf_model_t *model, int64_t idx);
uint64_t gguf_tensor_offset(const gguf_model_t *model, int64_t idx);
size_t gguf_tensor_nbytes(const gguf_model_t *model, int64_t idx);
size_t gguf_tensor_nbytes_pad(const gguf_model_t *model, int64_t idx);

/* replaces src/gguf_mmap.h:34-48: key/value metadata by index. gguf_kv_type gives the GGUF value type, or for an
 * array its element type. The scalar getters return 0, or -1 for an array, an absent index or a value the
 * requested type does not take (the same widening rules as the reference: e.g. u32 takes u8/i8/u16/i16/u32/i32,
 * f64 takes f32/f64, u8 takes a bool). */
int64_t gguf_n_kv(const gguf_model_t *model);
const char *gguf_kv_key(const gguf_model_t *model, int64_t idx);
int gguf_kv_type(const gguf_model_t *model, int64_t idx);
int32_t gguf_kv_get_u8(const gguf_model_t *model, int64_t idx, uint8_t *out);
int32_t gguf_kv_get_i8(const gguf_model_t *model, int64_t idx, int8_t *out);
int32_t gguf_kv_get_u16(const gguf_model_t *model, int64_t idx, uint16_t *out);
int32_t gguf_kv_get_i16(const gguf_model_t *model, int64_t idx, int16_t *out);
int32_t gguf_kv_get_u32(const gguf_model_t *model, int64_t idx, uint32_t *out);
int32_t gguf_kv_get_i32(const gguf_model_t *model, int64_t idx, int32_t *out);
int32_t gguf_kv_get_f32(const gguf_model_t *model, int64_t idx, float *out);
int32_t gguf_kv_get_u64(const gguf_model_t *model, int64_t idx, uint64_t *out);
int32_t gguf_kv_get_i64(const gguf_model_t *model, int64_t idx, int64_t *out);
int32_t gguf_kv_get_f64(const gguf_model_t *model, int64_t idx, double *out);

/* replaces src/gguf_mmap.h:51-71: file-level values and the model keys the engine reads ("<arch>.<suffix>"
 * first, then the reference's legacy key lists); absent keys give 0, "" or the default */
size_t gguf_alignment(const gguf_model_t *model);
size_t gguf_data_offset(const gguf_model_t *model);
uint32_t gguf_version(const gguf_model_t *model);
const char *gguf_arch(const gguf_model_t *model);
const char *gguf_vocab_name(const gguf_model_t *model);
const char *gguf_tokenizer_type(const gguf_model_t *model);
const char *gguf_pre_type(const gguf_model_t *model);
int64_t gguf_vocab_size(const gguf_model_t *model);
int64_t gguf_head_count(const gguf_model_t *model);
int64_t gguf_head_count_kv(const gguf_model_t *model);
int64_t gguf_context_length(const gguf_model_t *model);
int64_t gguf_embedding_length(const gguf_model_t *model);
int64_t gguf_block_count(const gguf_model_t *model);
int64_t gguf_arch_int(const gguf_model_t *model, const char *suffix, int64_t def);
float gguf_arch_float(const gguf_model_t *model, const char *suffix, float def);

/* replaces src/gguf_mmap.h:74-94: strings and arrays. Strings and string arrays are owned by the model
 * (gguf_free_string_array does nothing); numeric arrays point into the file mapping. */
const char *gguf_kv_str_val(const gguf_model_t *model, int64_t idx);
int32_t gguf_kv_get_string_array(const gguf_model_t *model, const char *key, const char ***out_strings,
                                 size_t *out_count);
void gguf_free_string_array(const char **strings, size_t count);
int32_t gguf_kv_get_array(const gguf_model_t *model, const char *key, int32_t *out_type, const void **out_data,
                          size_t *out_count);
int64_t gguf_find_kv(const gguf_model_t *model, const char *key);
int32_t gguf_kv_get_added_tokens(const gguf_model_t *model, const char *key, const char ***out_strings,
                                 size_t *out_count);

/* replaces src/gguf_mmap.h:96-118: a tensor's data by name (the staged copy once there is one: with
 * gguf_hbm_stage, a device address), the file mappings, gguf_remap (map whole pages of a mapping again in place;
 * 0 or -1), and the staging hooks */
const void *gguf_get_tensor_ptr(const gguf_model_t *model, const char *name, size_t *out_bytes);
const void *gguf_map_base(const gguf_model_t *model, size_t *out_size);
int gguf_n_maps(const gguf_model_t *model);
const void *gguf_map_at(const gguf_model_t *model, int i, size_t *out_size);
int gguf_remap(gguf_model_t *model, const void *p, size_t len);
const void *gguf_tensor_source(const gguf_model_t *model, int64_t idx);
int gguf_tensor_split(const gguf_model_t *model, int64_t idx);
void gguf_set_tensor_staged(gguf_model_t *model, int64_t idx, const void *p);
const char *gguf_file_path(const gguf_model_t *model, int i);
int gguf_file_identity(const gguf_model_t *model, int i, uint64_t out[4]);

/* replaces src/gguf_mmap.h:121: 1 for every block type (the reference's answer for all of them) */
int gguf_type_is_self_contained(int type);

/* ---- HBM residency (replaces src/model_stage.h:1-38 and pin_model_memory, src/inference.cpp:274): the
 * weights live in device memory instead of a pinned host mapping read over PCIe. ---- */

/* Device bytes gguf_hbm_stage needs for the tensors with keep[idx] != 0 (keep NULL: all), each at a 256-byte
 * aligned offset in index order; (size_t)-1 if one of them has an unknown size. */
size_t gguf_hbm_bytes(const gguf_model_t *model, const uint8_t *keep);

/* Copy those tensors into dev (caller-owned device memory of dev_bytes >= gguf_hbm_bytes) through pinned host
 * buffers, several host threads filling them while the previous chunk is in flight on stream, then point the
 * model at the copies (gguf_set_tensor_staged), so gguf_get_tensor_ptr / gguf_bind_weight return HBM addresses.
 * Returns when the copies are complete: 0, or -1 (nothing redirected). */
int gguf_hbm_stage(gguf_model_t *model, void *dev, size_t dev_bytes, const uint8_t *keep, hipStream_t stream);

/* replaces bind_weight (src/inference.cpp:362-389): a 2-D tensor (or 3-D expert stack, ne = {K, rows per expert,
 * experts}, bound as one matrix of ne[1] * ne[2] rows) of a type the matvecs take, its rows qt_row_size(type, K)
 * bytes each and the tensor exactly N of them. 0 bound, 1 absent, -1 unusable (type, shape or size). */
typedef struct {
    int type;
    int N, K;
    size_t row_bytes;
    const void *data;
} gguf_weight;
int gguf_bind_weight(const gguf_model_t *model, const char *name, gguf_weight *w);

#ifdef __cplusplus
}
#endif

#endif /* PURHIE_GGUF_MMAP_H */
