/*
 * C ABI of libunchain_kv_splitzip_cuda.so, the MI355X (gfx950) splitzip bf16
 * KV-cache codec.
 *
 * Every pointer, size and stream is passed as unsigned long long (a hipStream_t
 * for the stream; 0 is the null stream); every call only enqueues work on that
 * stream and returns without synchronising. Return convention (all functions
 * returning long long):
 *   > 0  bytes encoded / bytes written;
 *     0  declined: a precondition failed and nothing was launched (the caller
 *        falls back to another codec);
 *   < 0  a launch failed; the message is in kvq_splitzip_last_error().
 * Top-16 overflow is in-band: byte 0 of the payload is 255 once the stream has
 * run the encode.
 *
 * The first eight entry points have the names, argument order and meaning of the
 * reference library (native/unchain_kv/kvq_splitzip_cuda.cu); their comments cite
 * the function each one replaces. The rest are additions.
 */
#ifndef UNCHAIN_KV_SPLITZIP_H_
#define UNCHAIN_KV_SPLITZIP_H_

#ifdef __cplusplus
extern "C" {
#endif

/* Replaces kvq_splitzip_last_error (kvq_splitzip_cuda.cu:288): message of the last
 * failed call on this host thread. */
const char* kvq_splitzip_last_error(void);

/* Replaces kvq_splitzip_bf16_encode_mode (kvq_splitzip_cuda.cu:292). Palette encode
 * of `count` contiguous bf16 words at src into dst: bits 6 -> mode 3 (64-entry
 * palette), bits 5 -> mode 4 (32-entry). Returns the encoded size; 0 if bits is not
 * 5/6, if the encoded size is not below 2*count, or if capacity is smaller than
 * align4(encoded) + 1032 (scratch after the payload). The palette is ascending. */
long long kvq_splitzip_bf16_encode_mode(unsigned long long src_ptr, unsigned long long dst_ptr,
                                        unsigned long long count, unsigned long long capacity,
                                        unsigned long long stream_ptr, int bits);

/* Replaces kvq_splitzip_bf16_encode (kvq_splitzip_cuda.cu:335): encode_mode, bits 6. */
long long kvq_splitzip_bf16_encode(unsigned long long src_ptr, unsigned long long dst_ptr,
                                   unsigned long long count, unsigned long long capacity,
                                   unsigned long long stream_ptr);

/* Replaces kvq_splitzip_bf16_decode_fixed6_blocks (kvq_splitzip_cuda.cu:344). Decodes a
 * mode-3 payload of count_words = 2*block_count*block_words words and writes word i
 * to dst[p*plane_stride + blk*block_stride + within] (p = K/V plane, blk =
 * block_ids[j] or block_start + j when block_ids_ptr is 0). encoded_bytes must be
 * 65 + n + 3*ceil(n/4). Returns 2*count_words; a payload whose byte 0 is not 3 is
 * left unapplied. */
long long kvq_splitzip_bf16_decode_fixed6_blocks(
    unsigned long long src_ptr, unsigned long long encoded_bytes, unsigned long long dst_ptr,
    unsigned long long count_words, unsigned long long block_count,
    unsigned long long block_words, unsigned long long plane_stride,
    unsigned long long block_stride, unsigned long long block_start,
    unsigned long long block_ids_ptr, unsigned long long stream_ptr);

/* Replaces kvq_splitzip_bf16_decode_fixed6 (kvq_splitzip_cuda.cu:370): contiguous
 * block run starting at block_start. */
long long kvq_splitzip_bf16_decode_fixed6(
    unsigned long long src_ptr, unsigned long long encoded_bytes, unsigned long long dst_ptr,
    unsigned long long count_words, unsigned long long block_count,
    unsigned long long block_words, unsigned long long plane_stride,
    unsigned long long block_stride, unsigned long long block_start,
    unsigned long long stream_ptr);

/* Replaces kvq_splitzip_bf16_encode_top16 (kvq_splitzip_cuda.cu:381). Top-16 encode
 * (mode 5) of `count` contiguous bf16 words; the K/V split is at count/2. tables_ptr
 * is the 544-byte device table. Returns E = 5 + n + ceil(n/2) + 5*ceil(n/200); 0 if
 * count is 0 or above 2^32-1, if E >= 2*count, or if capacity < align4(E) + 8.
 * When capacity leaves room past the payload (16-byte aligned, 516 bytes per
 * 4096-word tile) the tiles are encoded in parallel using it as workspace;
 * otherwise they stage their escapes in their own body bytes, which a last pass
 * rewrites (one workgroup walks the tiles in order only for payloads whose
 * tiles hold fewer than 64 words). dst_ptr may be at any byte address. Escapes are
 * written in ascending position order and unused escape slots are zeroed. */
long long kvq_splitzip_bf16_encode_top16(unsigned long long src_ptr, unsigned long long dst_ptr,
                                         unsigned long long count, unsigned long long capacity,
                                         unsigned long long tables_ptr,
                                         unsigned long long stream_ptr);

/* Replaces kvq_splitzip_bf16_decode_top16_blocks (kvq_splitzip_cuda.cu:416). Decodes a
 * mode-5 payload and scatters it like decode_fixed6_blocks; escapes are applied in
 * any order. encoded_bytes must equal E(count_words). Returns 2*count_words; a
 * payload whose byte 0 is not 5 is left unapplied. */
long long kvq_splitzip_bf16_decode_top16_blocks(
    unsigned long long src_ptr, unsigned long long encoded_bytes, unsigned long long dst_ptr,
    unsigned long long count_words, unsigned long long block_count,
    unsigned long long block_words, unsigned long long plane_stride,
    unsigned long long block_stride, unsigned long long block_start,
    unsigned long long block_ids_ptr, unsigned long long tables_ptr,
    unsigned long long stream_ptr);

/* Replaces kvq_splitzip_bf16_decode_top16 (kvq_splitzip_cuda.cu:453): contiguous run. */
long long kvq_splitzip_bf16_decode_top16(
    unsigned long long src_ptr, unsigned long long encoded_bytes, unsigned long long dst_ptr,
    unsigned long long count_words, unsigned long long block_count,
    unsigned long long block_words, unsigned long long plane_stride,
    unsigned long long block_stride, unsigned long long block_start,
    unsigned long long tables_ptr, unsigned long long stream_ptr);

/* No counterpart in the reference: kvq_splitzip_bf16_decode_top16_blocks with the
 * block table in HOST memory (host_block_ids[0 .. block_count)), for callers whose
 * table is a host list (the reference's decode_top16 uploads it with torch.tensor
 * first, src/unchain_kv/splitzip_cuda.py:226-229). Up to 256 ids, each below 2^32,
 * travel in the kernel arguments, so no host-to-device copy precedes the launch;
 * the table is read before the call returns. Returns 0 (declined: use the
 * device-table entry) for more blocks or a geometry the tile kernels do not take
 * (block_words not a multiple of 1024, dst or strides off alignment). */
long long kvq_splitzip_bf16_decode_top16_host_blocks(
    unsigned long long src_ptr, unsigned long long encoded_bytes, unsigned long long dst_ptr,
    unsigned long long count_words, unsigned long long block_count,
    unsigned long long block_words, unsigned long long plane_stride,
    unsigned long long block_stride, const long long* host_block_ids,
    unsigned long long tables_ptr, unsigned long long stream_ptr);

/* No counterpart in the reference: kvq_splitzip_bf16_decode_fixed6_blocks with the
 * block table in host memory, under the same rules as
 * kvq_splitzip_bf16_decode_top16_host_blocks (the reference's decode_fixed6
 * uploads its list through the same _decode_layout). */
long long kvq_splitzip_bf16_decode_fixed6_host_blocks(
    unsigned long long src_ptr, unsigned long long encoded_bytes, unsigned long long dst_ptr,
    unsigned long long count_words, unsigned long long block_count,
    unsigned long long block_words, unsigned long long plane_stride,
    unsigned long long block_stride, const long long* host_block_ids,
    unsigned long long stream_ptr);

/* ------------------------------------------------------------------------------
 * Additions: every request of one paged layer in one launch.
 *
 * The reference gathers each request's blocks with torch.index_select into a packed
 * copy and then encodes that copy (src/unchain_kv/vllm_connector.py:2827-2869,
 * 3105); these entry points read the blocks in place through the block table and
 * handle all requests of a layer per launch (up to 64 payloads per launch, more in
 * several launches).
 *
 * Payload r consists of blocks block_ids[block_offsets[r] .. block_offsets[r+1]) of
 * the layer `kv` (words at kv[p*plane_stride + id*block_stride + w], w <
 * block_words); its n_r = 2*blocks_r*block_words words are ordered K then V, block
 * table order, then within the block, exactly as kv_layer[:, ids].contiguous().
 * block_offsets, out_offsets, src_offsets and encoded_bytes are HOST arrays;
 * block_ids is a DEVICE int64 array.
 * ---------------------------------------------------------------------------- */

/* Workspace bytes that kvq_splitzip_bf16_encode_top16_paged needs for this batch
 * (no counterpart in the reference). */
unsigned long long kvq_splitzip_top16_paged_workspace_bytes(
    unsigned long long block_words, const unsigned long long* block_offsets,
    unsigned long long payload_count);

/* Escape directory bytes of a batch (no counterpart in the reference): 68 bytes per
 * 4096-word tile of each plane of each payload, 0 when block_words is not a
 * multiple of 1024. The directory lists, per 1024-word chunk, where the chunk's
 * escapes sit in the payload's ascending escape list and the first three of them,
 * so that the decode applies escapes in its tile kernel instead of a second pass.
 * It is written by the encode below or built on the host by
 * kvq_splitzip_top16_build_directory; it is not part of the wire format. */
unsigned long long kvq_splitzip_top16_paged_directory_bytes(
    unsigned long long block_words, const unsigned long long* block_offsets,
    unsigned long long payload_count);

/* Gather + Top-16 encode (no counterpart in the reference; it replaces the
 * index_select + kvq_splitzip_bf16_encode_top16 pair per request). Payload r goes to
 * out + out_offsets[r]; payloads must not overlap and must fit in out_capacity.
 * workspace must hold kvq_splitzip_top16_paged_workspace_bytes() bytes.
 * directory_ptr: 0, or a 16-byte aligned device buffer of
 * kvq_splitzip_top16_paged_directory_bytes() bytes that receives the escape
 * directory (declined unless block_words is a multiple of 1024 and tables_ptr is
 * 4-byte aligned; payloads may start at any byte address). Returns the sum of the
 * encoded sizes, or 0 when a precondition fails. */
long long kvq_splitzip_bf16_encode_top16_paged(
    unsigned long long kv_ptr, unsigned long long plane_stride, unsigned long long block_stride,
    unsigned long long block_words, unsigned long long block_ids_ptr,
    const unsigned long long* block_offsets, unsigned long long payload_count,
    unsigned long long out_ptr, const unsigned long long* out_offsets,
    unsigned long long out_capacity, unsigned long long tables_ptr,
    unsigned long long workspace_ptr, unsigned long long workspace_bytes,
    unsigned long long directory_ptr, unsigned long long stream_ptr);

/* High-byte presence mask bytes of a batch (no counterpart in the reference): 32
 * bytes (a 256-bit mask of the high bytes present) per 4096-word tile of each plane
 * of each payload, payload r's masks after those of payloads 0 .. r-1; 0 when
 * block_words is not a multiple of 1024. */
unsigned long long kvq_splitzip_top16_paged_presence_bytes(
    unsigned long long block_words, const unsigned long long* block_offsets,
    unsigned long long payload_count);

/* kvq_splitzip_bf16_encode_top16_paged that also writes every tile's high-byte
 * presence mask to presence_ptr (16-byte aligned, kvq_splitzip_top16_paged_presence_bytes()
 * bytes; no counterpart in the reference). It is meant for a layer likely to
 * overflow: the palette fallback of an overflowed payload
 * (kvq_splitzip_bf16_encode_mode_paged_presence) then starts from the masks instead
 * of reading the payload's words a third time. Declined (0) under the directory's
 * conditions and when presence_ptr is 0. */
long long kvq_splitzip_bf16_encode_top16_paged_presence(
    unsigned long long kv_ptr, unsigned long long plane_stride, unsigned long long block_stride,
    unsigned long long block_words, unsigned long long block_ids_ptr,
    const unsigned long long* block_offsets, unsigned long long payload_count,
    unsigned long long out_ptr, const unsigned long long* out_offsets,
    unsigned long long out_capacity, unsigned long long tables_ptr,
    unsigned long long workspace_ptr, unsigned long long workspace_bytes,
    unsigned long long directory_ptr, unsigned long long presence_ptr,
    unsigned long long stream_ptr);

/* kvq_splitzip_bf16_encode_top16_paged_presence for a probe of a layer that
 * overflowed before (no counterpart in the reference; it replaces the Top-16 attempt
 * of the reference connector's probe, vllm_connector.py:3078-3123, whose overflowed
 * payload is re-encoded as fixed6, :4557-4633). In the same launch as its finalize it
 * also writes each payload's palette record (512 bytes: 256-bit presence mask,
 * distinct count, rank table, ascending palette) to palette_info_ptr + 512 r
 * (16-byte aligned, payload_count records), which
 * kvq_splitzip_bf16_encode_mode_paged_info takes instead of a presence and reduce
 * pass; and a payload found to overflow gets its header (255, count clamped to the
 * capacity), body and codes but no escape placement: its escape section stays zero
 * (the reference's holds escapes in atomic order, and both are discarded for the
 * fixed6 re-encode). Payloads that fit are byte-identical to the plain encode's.
 * Declined (0) when presence_ptr or palette_info_ptr is 0, and as the presence
 * variant. */
long long kvq_splitzip_bf16_encode_top16_paged_probe(
    unsigned long long kv_ptr, unsigned long long plane_stride, unsigned long long block_stride,
    unsigned long long block_words, unsigned long long block_ids_ptr,
    const unsigned long long* block_offsets, unsigned long long payload_count,
    unsigned long long out_ptr, const unsigned long long* out_offsets,
    unsigned long long out_capacity, unsigned long long tables_ptr,
    unsigned long long workspace_ptr, unsigned long long workspace_bytes,
    unsigned long long directory_ptr, unsigned long long presence_ptr,
    unsigned long long palette_info_ptr, unsigned long long stream_ptr);

/* No counterpart in the reference: kvq_splitzip_bf16_encode_top16_paged for callers
 * that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Same arguments, results and preconditions,
 * without the workspace: the escape staging lives in a fixed array of
 * kvq_splitzip_top16_noalloc_scratch_bytes() bytes (16 MiB) per GPU, owned by the
 * library for the life of the process; the call allocates nothing. A batch that
 * needs more than that (kvq_splitzip_top16_paged_workspace_bytes) returns -1 with
 * the reason in kvq_splitzip_last_error(). Every call on one GPU shares the array:
 * calls that overlap on one GPU (different streams, or different host threads)
 * race and must be serialised by the caller. */
long long kvq_splitzip_bf16_encode_top16_paged_noalloc(
    unsigned long long kv_ptr, unsigned long long plane_stride, unsigned long long block_stride,
    unsigned long long block_words, unsigned long long block_ids_ptr,
    const unsigned long long* block_offsets, unsigned long long payload_count,
    unsigned long long out_ptr, const unsigned long long* out_offsets,
    unsigned long long out_capacity, unsigned long long tables_ptr,
    unsigned long long directory_ptr, unsigned long long stream_ptr);

/* Size of the fixed per-GPU scratch of kvq_splitzip_bf16_encode_top16_paged_noalloc
 * (no counterpart in the reference). */
unsigned long long kvq_splitzip_top16_noalloc_scratch_bytes(void);

/* Top-16 decode + scatter of a batch (no counterpart in the reference; it replaces one
 * kvq_splitzip_bf16_decode_top16_blocks call per request). Payload r is read from
 * src + src_offsets[r] and must be encoded_bytes[r] = E(n_r) long; it is written into
 * the blocks of block table r. directory_ptr: 0 (escapes applied by a second
 * kernel, in any order), or the escape directory of these payloads (from their
 * encode with the same block counts, or kvq_splitzip_top16_build_directory), with
 * the conditions of the encode; the decode is then one kernel. Returns the total
 * raw bytes (sum of 2*n_r). */
long long kvq_splitzip_bf16_decode_top16_paged(
    unsigned long long src_ptr, const unsigned long long* src_offsets,
    const unsigned long long* encoded_bytes, unsigned long long payload_count,
    unsigned long long kv_ptr, unsigned long long plane_stride, unsigned long long block_stride,
    unsigned long long block_words, unsigned long long block_ids_ptr,
    const unsigned long long* block_offsets, unsigned long long tables_ptr,
    unsigned long long directory_ptr, unsigned long long stream_ptr);

/* Host-side escape directory of Top-16 payloads held in HOST memory (no counterpart
 * in the reference): payload r at host_buf + offsets[r] (encoded_bytes[r] long, of
 * the batch's block counts). Sorts each mode-5 payload's escape list by position in
 * place (the decode's result does not depend on that order) and writes the
 * directory (kvq_splitzip_top16_paged_directory_bytes() bytes) to host_directory,
 * to be copied to the device with the payloads. Returns the directory bytes, or 0
 * when block_words is not a multiple of 1024, directory_bytes is too small or a
 * size is not E(n_r). */
long long kvq_splitzip_top16_build_directory(
    unsigned char* host_buf, const unsigned long long* offsets,
    const unsigned long long* encoded_bytes, unsigned long long payload_count,
    unsigned long long block_words, const unsigned long long* block_offsets,
    unsigned char* host_directory, unsigned long long directory_bytes);

/* Workspace bytes that kvq_splitzip_bf16_encode_mode_paged needs for this batch (no
 * counterpart in the reference). */
unsigned long long kvq_splitzip_palette_paged_workspace_bytes(
    unsigned long long block_words, const unsigned long long* block_offsets,
    unsigned long long payload_count);

/* Gather + palette encode of a batch: bits 6 -> fixed6 (mode 3), bits 5 -> fixed5
 * (mode 4) (no counterpart in the reference; it replaces index_select +
 * kvq_splitzip_bf16_encode_mode per request, the connector's Top-16 overflow
 * fallback, vllm_connector.py:4557-4616). Payload r goes to out + out_offsets[r];
 * each payload gets its own ascending palette, or byte 0 = 255 alone when its
 * distinct high bytes exceed the palette. workspace (16-byte aligned) must hold
 * kvq_splitzip_palette_paged_workspace_bytes() bytes. Returns the sum of the
 * encoded sizes, or 0 when a precondition fails. */
long long kvq_splitzip_bf16_encode_mode_paged(
    unsigned long long kv_ptr, unsigned long long plane_stride, unsigned long long block_stride,
    unsigned long long block_words, unsigned long long block_ids_ptr,
    const unsigned long long* block_offsets, unsigned long long payload_count,
    unsigned long long out_ptr, const unsigned long long* out_offsets,
    unsigned long long out_capacity, unsigned long long workspace_ptr,
    unsigned long long workspace_bytes, unsigned long long stream_ptr, int bits);

/* kvq_splitzip_bf16_encode_mode_paged with the high-byte presence masks already
 * known (no counterpart in the reference): payload r's masks, one per 4096-word tile
 * of each of its planes, start at mask presence_first[r] (a HOST array) of
 * presence_ptr (a device buffer written by kvq_splitzip_bf16_encode_top16_paged_presence
 * over the same blocks; 16-byte aligned), so the encode skips its presence pass.
 * Same results and other preconditions. */
long long kvq_splitzip_bf16_encode_mode_paged_presence(
    unsigned long long kv_ptr, unsigned long long plane_stride, unsigned long long block_stride,
    unsigned long long block_words, unsigned long long block_ids_ptr,
    const unsigned long long* block_offsets, unsigned long long payload_count,
    unsigned long long out_ptr, const unsigned long long* out_offsets,
    unsigned long long out_capacity, unsigned long long workspace_ptr,
    unsigned long long workspace_bytes, unsigned long long presence_ptr,
    const unsigned long long* presence_first, unsigned long long stream_ptr, int bits);

/* kvq_splitzip_bf16_encode_mode_paged from the palette records of a Top-16 probe
 * encode (no counterpart in the reference): payload r's palette is record
 * info_first[r] (a HOST array, each < info_count) of info_ptr (written by
 * kvq_splitzip_bf16_encode_top16_paged_probe over the same blocks; 16-byte aligned);
 * no workspace, presence or reduce pass. Same results and other preconditions;
 * declined (0) for block geometries the tile kernels do not take. */
long long kvq_splitzip_bf16_encode_mode_paged_info(
    unsigned long long kv_ptr, unsigned long long plane_stride, unsigned long long block_stride,
    unsigned long long block_words, unsigned long long block_ids_ptr,
    const unsigned long long* block_offsets, unsigned long long payload_count,
    unsigned long long out_ptr, const unsigned long long* out_offsets,
    unsigned long long out_capacity, unsigned long long info_ptr,
    const unsigned long long* info_first, unsigned long long info_count,
    unsigned long long stream_ptr, int bits);

/* Palette decode + scatter of a batch (no counterpart in the reference; it replaces
 * one kvq_splitzip_bf16_decode_fixed6_blocks call per request, and decodes fixed5 on
 * the GPU where the reference uses torch ops). Payload r (src + src_offsets[r],
 * encoded_bytes[r] long, which must be the format's exact size) is written into the
 * blocks of block table r; a payload whose byte 0 is not the format's mode byte is
 * left unapplied. Returns the total raw bytes. */
long long kvq_splitzip_bf16_decode_mode_paged(
    unsigned long long src_ptr, const unsigned long long* src_offsets,
    const unsigned long long* encoded_bytes, unsigned long long payload_count,
    unsigned long long kv_ptr, unsigned long long plane_stride, unsigned long long block_stride,
    unsigned long long block_words, unsigned long long block_ids_ptr,
    const unsigned long long* block_offsets, unsigned long long stream_ptr, int bits);

/* Decode + scatter of the reference connector's torch-op codec payloads, modes 0
 * (palette of high bytes), 1 (four nibble planes) and 2 (sign/magnitude), mixed
 * in one batch (no counterpart in the reference library: it replaces the torch
 * decoders of _copy_splitzip_bf16_native_blocks, src/unchain_kv/vllm_connector.py:
 * 5168-5252, followed by index_copy_). Payload r (src + src_offsets[r],
 * encoded_bytes[r] long) goes into the blocks of block table r; a payload whose
 * header does not give exactly its encoded size is left unapplied. Returns the
 * total raw bytes. */
long long kvq_splitzip_bf16_decode_torchop_paged(
    unsigned long long src_ptr, const unsigned long long* src_offsets,
    const unsigned long long* encoded_bytes, unsigned long long payload_count,
    unsigned long long kv_ptr, unsigned long long plane_stride, unsigned long long block_stride,
    unsigned long long block_words, unsigned long long block_ids_ptr,
    const unsigned long long* block_offsets, unsigned long long stream_ptr);

/* Torch-op encode of a batch, in two calls with a host read between them (no
 * counterpart in the reference library: it replaces the torch ops of
 * _splitzip_bf16_native_blocks, src/unchain_kv/vllm_connector.py:3204-3343, which a
 * sender takes for a request below 1 MiB without Top-16 native decode, :3043-3046).
 *
 * kvq_splitzip_bf16_plan_torchop_paged writes one 64-byte plan record per payload
 * to plans (device, 8-byte aligned):
 *   bytes  0-31  256-bit presence mask of the words' high bytes
 *   bytes 32-35  presence of the values of bits 0-3 (bits 0-15) and bits 4-7
 *                (bits 16-31)
 *   byte  36     mode the reference picks: 2 (sign/magnitude) when the magnitudes
 *                span fewer than 7 bits and the payload is smaller than the raw
 *                words, else 0 (high-byte palette) when it has at most 128 entries
 *                and is smaller, else 1 (nibble planes) when smaller, else 255
 *   bytes 37-40  widths (modes 2, 0: byte 37; mode 1: one per nibble plane)
 *   byte  41     smallest magnitude (mode 2)
 *   bytes 48-55  encoded bytes (u64; 0 when declined), bytes 56-63 words n
 * workspace: kvq_splitzip_torchop_workspace_bytes() bytes of device memory.
 * Returns payload_count, or 0 on a failed precondition.
 *
 * kvq_splitzip_bf16_encode_torchop_paged then writes payload r, as the reference's
 * encoder writes it, to out + out_offsets[r]; encoded_bytes[r] is its plan's size
 * (0: declined, nothing written). A payload whose plan in device memory does not
 * give that size is not written. Returns the total encoded bytes, 0 on a failed
 * precondition, -1 on a launch error. Block tables as in the batched decode. */
unsigned long long kvq_splitzip_torchop_plan_bytes(void);
unsigned long long kvq_splitzip_torchop_workspace_bytes(
    unsigned long long block_words, const unsigned long long* block_offsets,
    unsigned long long payload_count);
long long kvq_splitzip_bf16_plan_torchop_paged(
    unsigned long long kv_ptr, unsigned long long plane_stride, unsigned long long block_stride,
    unsigned long long block_words, unsigned long long block_ids_ptr,
    const unsigned long long* block_offsets, unsigned long long payload_count,
    unsigned long long workspace_ptr, unsigned long long workspace_bytes,
    unsigned long long plans_ptr, unsigned long long stream_ptr);
long long kvq_splitzip_bf16_encode_torchop_paged(
    unsigned long long kv_ptr, unsigned long long plane_stride, unsigned long long block_stride,
    unsigned long long block_words, unsigned long long block_ids_ptr,
    const unsigned long long* block_offsets, unsigned long long payload_count,
    unsigned long long plans_ptr, unsigned long long out_ptr,
    const unsigned long long* out_offsets, const unsigned long long* encoded_bytes,
    unsigned long long out_capacity, unsigned long long stream_ptr);

/* ------------------------------------------------------------------------------
 * bf16 exponent histograms of a paged layer: the statistics Top-16 codebooks are
 * fit from (no counterpart in the reference as a native call: it runs
 * torch.bincount((word >> 7) & 0xFF) per plane of a gathered request,
 * src/unchain_kv/vllm_connector.py:2871-2904, and ranks the counts offline,
 * scripts/extract_llama_top16_codebooks.py:15-60).
 * ---------------------------------------------------------------------------- */

/* Workspace bytes kvq_splitzip_exponent_histogram_paged needs. */
unsigned long long kvq_splitzip_exponent_histogram_workspace_bytes(
    unsigned long long block_count, unsigned long long block_words);

/* counts (device, 512 x u64, overwritten): [b] = K-plane words of blocks
 * ids[0 .. block_count) whose exponent bits (word >> 7) & 0xFF equal b, [256 + b]
 * the same for the V plane. block_ids_ptr: device int64 array; plane_stride and
 * block_stride in elements. Returns the words counted (2 * block_count *
 * block_words), 0 on a failed precondition. Deterministic (no global atomics). */
long long kvq_splitzip_exponent_histogram_paged(
    unsigned long long kv_ptr, unsigned long long plane_stride, unsigned long long block_stride,
    unsigned long long block_words, unsigned long long block_ids_ptr,
    unsigned long long block_count, unsigned long long counts_ptr,
    unsigned long long workspace_ptr, unsigned long long workspace_bytes,
    unsigned long long stream_ptr);

/* ------------------------------------------------------------------------------
 * Codec writeback: encoded payloads moved into the sending request's own KV
 * blocks so the codec buffer is free before the host copy (replaces the two
 * segment copies per request of _try_splitzip_writeback,
 * src/unchain_kv/vllm_connector.py:3460-3563, segments from
 * _kv_writeback_segments :3720-3738).
 * ---------------------------------------------------------------------------- */

/* For r < payload_count: if byte 0 of payload r (payloads_ptr +
 * payload_offsets[r], encoded_bytes[r] bytes) is 5, its bytes are written to the
 * K-plane run of blocks [run_starts[r], run_starts[r] + run_blocks[r]) and, past
 * that run's 2 * run_blocks[r] * block_words bytes, to the V-plane run of the same
 * blocks (kv_ptr: bf16 layer, plane_stride and block_stride in elements; a run of
 * several blocks needs block_stride == block_words). Any other mode byte (255, an
 * overflow) leaves the blocks unchanged. status_ptr: device u8 array, [r] = byte 0
 * of payload r. Host arrays of payload_count entries. Returns the sum of
 * encoded_bytes, 0 on a failed precondition (a payload longer than its two runs,
 * runs overlapping each other or the payload range), -1 on a launch error. */
long long kvq_splitzip_top16_writeback_paged(
    unsigned long long payloads_ptr, const unsigned long long* payload_offsets,
    const unsigned long long* encoded_bytes, unsigned long long payload_count,
    unsigned long long kv_ptr, unsigned long long plane_stride, unsigned long long block_stride,
    unsigned long long block_words, const unsigned long long* run_starts,
    const unsigned long long* run_blocks, unsigned long long status_ptr,
    unsigned long long stream_ptr);

/* ------------------------------------------------------------------------------
 * Fused Top-16 decode + decode attention (no counterpart in the reference, whose
 * consumer decodes each payload into the paged KV cache and then runs attention;
 * scripts/bench_codec_attention.py times that pairing).
 *
 * One query token per sequence. Sequence r's KV is the Top-16 payload (mode 5) at
 * payloads + payload_offsets[r] of its block table in token order: span_r =
 * ceil(context_tokens[r] / block_tokens) * block_tokens tokens, its K plane then
 * its V plane, words ordered [token][kv head][dim] (the batched encoder's payload
 * of the table, block = (block_tokens, kv heads, head_dim)); attention covers the
 * first context_tokens[r] tokens. q and out are bf16 [batch][q_heads][head_dim]
 * device arrays; tables_ptr is the layer's 544-byte table. Requires head_dim 128,
 * q_heads = 4 * kv_heads (GQA groups of 4), escapes in ascending order (this
 * library's encoder), body sections 16-byte aligned ((payloads + offset + 5) % 16
 * == 0) and 2 * span_r * kv_heads * 128 < 2^32. payload_offsets and context_tokens
 * are HOST arrays of batch entries.
 * A payload whose byte 0 is not 5, or whose escapes are found out of order, gives
 * NaN outputs for its heads. Returns the bytes of out, or 0 when a precondition
 * fails.
 * ---------------------------------------------------------------------------- */

/* Workspace bytes kvq_splitzip_top16_decode_attention needs (split partials). */
unsigned long long kvq_splitzip_top16_decode_attention_workspace_bytes(
    unsigned long long batch, unsigned long long kv_heads, unsigned long long max_ctx);

long long kvq_splitzip_top16_decode_attention(
    unsigned long long q_ptr, unsigned long long out_ptr, unsigned long long payloads_ptr,
    const unsigned long long* payload_offsets, const unsigned long long* context_tokens,
    unsigned long long block_tokens, unsigned long long batch, unsigned long long q_heads,
    unsigned long long kv_heads, unsigned long long head_dim, unsigned long long tables_ptr,
    unsigned long long workspace_ptr, unsigned long long workspace_bytes, float scale,
    unsigned long long stream_ptr);

#ifdef __cplusplus
}
#endif

#endif /* UNCHAIN_KV_SPLITZIP_H_ */
