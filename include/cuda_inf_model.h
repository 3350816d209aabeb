/*
 * cuda_inf_model.h -- C-ABI of the model files around the attention path:
 * the weight index (index.bin), the weight blob (weights.bin) uploaded to
 * HBM, and the byte-level BPE tokenizer (tok/vocab.tsv, merges.tsv,
 * special.tsv).  Same conventions as cuda_inf_attn.h: every entry returns
 * CIA_OK or a cia_status code (CIA_ERR_IO for a file that cannot be opened,
 * read or parsed) and none calls exit().
 *
 * File formats (the reference's exporters write them):
 *   index.bin  little-endian: u32 count, then per tensor u8 name_len, name
 *              bytes, u8 kind (0 fp16, 1 int4g), u64 offset, u64 packed,
 *              u64 scales, i64 d0, i64 d1          (tools/make_index.py:3-11)
 *   weights.bin  the tensors' bytes at their offsets; an int4g tensor holds
 *              `packed` bytes of nibbles (N x K/2) then `scales` bytes of
 *              fp16 group scales (N x K/128)       (tools/export_weights.py:1-13)
 *   tok/vocab.tsv    "<id>\t<byte-level token>"  one per line
 *   tok/merges.tsv   "<rank>\t<A>\t<B>"          lower rank merges first
 *   tok/special.tsv  "<id>\t<content>"           matched literally
 *                                                (tools/export_tokenizer.py:1-9)
 */
#ifndef CUDA_INF_MODEL_H
#define CUDA_INF_MODEL_H

#include <stdint.h>

#include "cuda_inf_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* One index entry.  name is NUL-terminated (index names are at most 255
 * bytes).  For kind 0 (fp16) `packed` is the data size and `scales` 0. */
typedef struct cia_tensor_desc {
  char name[256];
  int32_t kind;
  uint64_t offset, packed, scales;
  int64_t d0, d1;
} cia_tensor_desc;

/* Parses index.bin at `path` (host memory only).  *count receives the
 * number of tensors; with out == NULL (cap ignored) that is all it does,
 * else out[0..count) are filled and cap < count is CIA_ERR_ARG.  A short
 * file, an unknown kind or trailing bytes are CIA_ERR_IO.
 * Replaces the index loop of main() (src/engine.cu:665-675). */
int cia_index_read(const char* path, cia_tensor_desc* out, int64_t cap, int64_t* count);

/* Size in bytes of the file at `path` (the device blob to allocate for
 * cia_weights_upload). */
int cia_file_size(const char* path, uint64_t* bytes);

/* Copies the whole file at `path` into device memory `dst` (cap bytes
 * available; a larger file is CIA_ERR_ARG) on `stream`, and returns once
 * the bytes are in HBM (*nbytes = file size).  The file is read by up to
 * 12 host threads into two pinned staging buffers (allocated per call,
 * 2 x 64 MiB), each buffer's copy overlapping the next buffer's reads.
 * Replaces the blob upload of main() (src/engine.cu:678-692: one pageable
 * 256 MiB buffer, read and copied in turn). */
int cia_weights_upload(const char* path, void* dst, uint64_t cap, uint64_t* nbytes,
                       void* stream);

/* The tokenizer (host only). */
typedef struct cia_tokenizer cia_tokenizer;

/* Loads <dir>/vocab.tsv, merges.tsv and special.tsv; a missing file is
 * CIA_ERR_IO and *out stays NULL.  Special tokens with empty content are
 * ignored (an empty literal would match everywhere).
 * Replaces Tokenizer::load (src/tokenizer.h:42-81). */
int cia_tok_load(const char* dir, cia_tokenizer** out);
void cia_tok_free(cia_tokenizer* tok);

/* Token ids of the `len` bytes at `text` (UTF-8; the text is split at
 * special tokens, pre-tokenized GPT-2 style, byte-level mapped and BPE
 * merged).  *n receives the count; at most `len` ids are produced, so
 * cap >= len always suffices; with ids == NULL only *n is set, else a
 * smaller cap than *n is CIA_ERR_ARG.
 * Replaces Tokenizer::encode (src/tokenizer.h:177-208). */
int cia_tok_encode(const cia_tokenizer* tok, const char* text, int64_t len, int32_t* ids,
                   int64_t cap, int64_t* n);

/* The bytes of `n` token ids (special tokens as their content unless
 * skip_special; ids outside the vocabulary are skipped).  *len receives
 * the byte count; with out == NULL only *len is set, else a smaller cap
 * than *len is CIA_ERR_ARG.  No NUL is appended.
 * Replaces Tokenizer::decode (src/tokenizer.h:218-231). */
int cia_tok_decode(const cia_tokenizer* tok, const int32_t* ids, int64_t n, int skip_special,
                   char* out, int64_t cap, int64_t* len);

#ifdef __cplusplus
}
#endif

#endif /* CUDA_INF_MODEL_H */
