/* libcfattn.so -- the on-disk formats of a cpuforge training run, read into
 * and written from HBM-resident tensors (AMD MI355X, gfx950).
 *
 * The reference keeps resumable training state and LoRA adapters in
 * safetensors files (crates/io/src/st.rs, train/src/state.rs,
 * io/src/hf.rs) through the `safetensors` crate 0.8.0 (Cargo.lock:1177-1178).
 * With the model's parameters and optimizer moments held on the GPU, the
 * file's tensor bytes move between the file and HBM here: through two pinned
 * host staging chunks, each H2D/D2H copy overlapped with the file read or
 * write of the other chunk, and bf16 / f16 tensors are widened to f32 on the
 * GPU after the copy (half the bytes over the bus).  The file layout is the
 * crate's: an 8-byte little-endian header length, a JSON header
 * ({"__metadata__":{...}, name:{"dtype","shape","data_offsets"}}, tensors in
 * the crate's order, padded with spaces to a multiple of 8 bytes), then the
 * tensor bytes.  Files written here are byte-identical to what the crate
 * writes for the same tensors and metadata (its metadata keys come in hash
 * order, written here in sorted order).
 *
 * Reference sources (Sm0r3s-source/cpuforge, crates/...):
 *   io/src/dtype.rs:3-33     bf16_to_f32 / f16_to_f32
 *   io/src/st.rs:19-45       read_safetensors
 *   io/src/st.rs:48-64       write_safetensors (temp file, then rename)
 *
 * Status codes and messages are those of include/cfattn.h; entry points that
 * take no context write their message into a caller buffer instead.
 */
#ifndef CFIO_H
#define CFIO_H

#include <stddef.h>
#include <stdint.h>

#include "cfattn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Element types of a safetensors header, in the crate's `Dtype` order
 * (safetensors 0.8.0, tensor.rs): the writer sorts tensors by this order,
 * descending, then by name. Only F32, BF16 and F16 tensors can be read into
 * f32 (io/src/st.rs:36-41); the others are reported as unsupported. */
enum {
    CFIO_BOOL = 0, CFIO_F4, CFIO_F6_E2M3, CFIO_F6_E3M2, CFIO_U8, CFIO_I8, CFIO_F8_E5M2, CFIO_F8_E4M3, CFIO_F8_E8M0,
    CFIO_I16, CFIO_U16, CFIO_F16, CFIO_BF16, CFIO_I32, CFIO_U32, CFIO_F32, CFIO_C64, CFIO_F64, CFIO_I64, CFIO_U64,
    CFIO_NUM_DTYPES
};

/* dtype.rs:3-5 and 7-33 on the device: dst[i] = the f32 value of the 16-bit
 * pattern src[i].  Exact for every pattern (f16 subnormals renormalised,
 * inf and NaN payloads kept bit for bit).  Queued on `stream`. */
int cfio_bf16_to_f32(cfattn_ctx* ctx, const uint16_t* src, float* dst, size_t n, void* stream);
int cfio_f16_to_f32(cfattn_ctx* ctx, const uint16_t* src, float* dst, size_t n, void* stream);

/* An open safetensors file: its parsed and validated header.  The checks are
 * the crate's `SafeTensors::deserialize` (header length within the file and
 * at most 100,000,000 bytes, a JSON object, offsets that tile the data section
 * from 0 with no gap or overlap, each tensor's byte length equal to its
 * element count times its dtype size).  Needs no GPU. */
typedef struct cfio_file cfio_file;

/* read_safetensors's open and parse (st.rs:19-33).  On failure *out is NULL
 * and `err` (when non-NULL, `err_cap` bytes) holds "cannot open PATH: ..." or
 * "PATH: <what is wrong with the header>". */
int cfio_st_open(const char* path, cfio_file** out, char* err, size_t err_cap);
int cfio_st_close(cfio_file* f);

/* Tensors, in file order (by data offset).  `name` and `shape` stay valid
 * until cfio_st_close; `dtype` is a CFIO_* code. */
size_t cfio_st_count(const cfio_file* f);
int cfio_st_tensor(const cfio_file* f, size_t i, const char** name, int* dtype, size_t* ndim, const size_t** shape,
                   size_t* numel);
/* Index of the tensor called `name`, or -1. */
long long cfio_st_find(const cfio_file* f, const char* name);
/* The "__metadata__" string map, in header order. */
size_t cfio_st_meta_count(const cfio_file* f);
int cfio_st_meta(const cfio_file* f, size_t i, const char** key, const char** value);
const char* cfio_dtype_name(int dtype); /* "F32", "BF16", ... as the crate names them */

/* read_safetensors's conversion (st.rs:34-43), into HBM: tensor idx[j] of
 * the file goes to dst[j], a device buffer of its element count in f32,
 * widened from bf16 or f16 on the GPU.  A tensor of any other dtype is
 * CFATTN_ERR_ARG "tensor 'NAME' has unsupported dtype I64" and nothing is
 * read.  The copies are queued on `stream`; the call returns once the file's
 * bytes are in the context's staging buffers (the file may be closed then). */
int cfio_st_read_f32(cfattn_ctx* ctx, const cfio_file* f, size_t count, const size_t* idx, float* const* dst,
                     void* stream);

/* write_safetensors (st.rs:48-64) from HBM: `count` f32 tensors, tensor j
 * called names[j] with shape shapes[j][0..ndims[j]) and data the device
 * buffer data[j]; `n_meta` metadata pairs (none: no "__metadata__" entry, as
 * the reference passes None for an empty map).  Waits for `stream` (the data
 * are read after the work queued before the call), writes PATH with its
 * extension replaced by "tmp" and renames that file to PATH.  Errors: "cannot
 * write PATH: ..." and "cannot move TMP into place: ...". */
int cfio_st_write(cfattn_ctx* ctx, const char* path, size_t count, const char* const* names, const size_t* ndims,
                  const size_t* const* shapes, const float* const* data, size_t n_meta, const char* const* keys,
                  const char* const* values, void* stream);

/* Size of each of the two pinned staging chunks (default 8 MiB, at least
 * 1 MiB); the device side holds two chunks of the same size.  A chunk's file
 * ranges are read by a pool of eight threads and the caller's. */
int cfio_set_chunk_bytes(cfattn_ctx* ctx, size_t bytes);

#ifdef __cplusplus
}
#endif
#endif
