/*
 * daser_kv.h -- C ABI of the MI355X (gfx950) KV data-movement library
 * (libdaser_kv.so).
 *
 * The library moves vLLM paged-KV pages between the per-layer block cache and
 * contiguous DaseR slot records, and optionally re-rotates the K half of
 * reused chunks to a new RoPE position while scattering them back.
 *
 * Byte layouts (all offsets in bytes):
 *   per-layer block cache  kv_l[2][num_blocks][block_size][H][D]  (index 0 = K)
 *       K page of block b  = layer_base[l] + b * page_stride
 *       V page of block b  = layer_base[l] + b * page_stride + kv_stride
 *       page_bytes         = block_size * H * D * elem_bytes (contiguous)
 *   slot record            = [layer 0: K page | V page][layer 1: ...]...
 *       record of (page p, layer l) starts at
 *           staging + slot_offsets[p] + l * layer_bytes
 *       K page first, V page at + page_bytes; layer_bytes >= 2 * page_bytes.
 *   This is the on-disk `daser.store` slot format of the reference
 *   (daser/connector/daser_connector.py:531-535, :625-632; SLOT = LAYER * L,
 *   LAYER = kv.nbytes // num_blocks, :404-408).
 *
 * Conventions for every entry point:
 *   - pointer arguments marked [device] are device addresses; the tables they
 *     point to must be resident before the stream reaches the launch;
 *   - every base pointer, stride, page_bytes, layer_bytes and slot offset
 *     must be a multiple of 16 bytes (one 16-byte lane vector); violations
 *     return DSR_ERR_ALIGN without launching;
 *   - launches are stream-ordered on `stream` (0 = the null stream), never
 *     synchronise, never allocate, and are reentrant across streams;
 *   - pages whose block id lies outside [0, num_blocks), or whose record
 *     would end beyond staging_bytes, are skipped by the kernel, never
 *     touched and not reported (the Python wrappers reject them in host
 *     tables before launching; daser_amd.ops.check_tables checks
 *     device-resident ones on request);
 *   - return value: 0 on success, a DSR_ERR_* code (< 0) for argument errors,
 *     or a positive hipError_t from the launch.
 */
#ifndef DASER_KV_H
#define DASER_KV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* dsr_stream_t; /* == hipStream_t */

/* Bumped whenever an entry point's signature changes or one is added:
 * 2 layer_group on the re-rotation, 3 dsr_scatter_rerotate_kx, 4 the
 * re-rotations' flags, 5 the head-major (_hnd) entry points, 6
 * dsr_set_tuning, 7 dsr_scatter_ex, 8 dsr_scatter_slots_rerotate, 9
 * DSR_RING_MMAP and dsr_ring_is_mapped, 10 dsr_scatter_rerotate_static, 11
 * dsr_scatter_fanout. Callers check dsr_abi_version() against it. */
#define DSR_ABI_VERSION 11

/*
 * Kernel choice and launch shape follow from the geometry. dsr_set_tuning()
 * overrides them for measurements and tests only (results are the same
 * bytes); the library reads no environment variables. Knobs (value 0 = the
 * geometry's own choice):
 *   DSR_TUNE_UNITS_PER_GROUP      cap the (page, layer) units per workgroup
 *                                 of the small-page kernels (1: off)
 *   DSR_TUNE_MAX_WG_PER_LAUNCH    split calls into launches of <= n workgroups
 *   DSR_TUNE_ROT_KERNEL           re-rotation kernel where several apply:
 *                                 1 pairs, 2 contig, 3 grouped
 *   DSR_TUNE_ROT_WG_PER_CU, DSR_TUNE_ROT_GROUPED_WG_PER_CU
 *                                 re-rotation occupancy
 *   DSR_TUNE_SLOTS_TPW            4|8|16 tokens per wave of the small-row
 *                                 token kernels
 *   DSR_TUNE_SLOTS_KERNEL         1: rows of <= 8 vectors take the small-row
 *                                 kernel instead of the packed one
 *   DSR_TUNE_SLOTS_UNROLL         4|8 instructions per wave of the packed kernel
 *   DSR_TUNE_COPY_WG_PER_CU       workgroups per CU of the one-unit page
 *                                 gather / scatter
 *   DSR_TUNE_SCATTER_KERNEL       one-unit page scatter: 1 the load-all-then-
 *                                 store kernel, 2 the streaming kernel in
 *                                 hardware dispatch order, 3 the streaming
 *                                 kernel in per-XCD layer-major order
 *                                 (streaming: pages of 16 KiB multiples)
 *   DSR_TUNE_GATHER_SPLIT         workgroups per (page, layer) unit of a
 *                                 one-unit page gather (1: no split)
 *   DSR_TUNE_PAGE_PARTS           parts (one workgroup each) of a page in
 *                                 the one-unit gather and streaming scatter
 *                                 (1: whole pages; default: 32 KiB parts of
 *                                 larger pages)
 *   DSR_TUNE_SLOTS_ORDER          unit order of the large-row token scatters
 *                                 (plain and re-rotating): 1 per-XCD
 *                                 layer-major, 2 layer-major in hardware
 *                                 dispatch order
 *   DSR_TUNE_SLOTS_WG_PER_CU      workgroups per CU of those kernels
 *   DSR_TUNE_FANOUT_WG_PER_CU     workgroups per CU of dsr_scatter_fanout
 *   DSR_TUNE_FANOUT_PARTS         workgroups per (record, layer) unit of
 *                                 dsr_scatter_fanout (1, 2, 4: parts of
 *                                 whole rows)
 */
#define DSR_TUNE_UNITS_PER_GROUP 0
#define DSR_TUNE_MAX_WG_PER_LAUNCH 1
#define DSR_TUNE_ROT_KERNEL 2
#define DSR_TUNE_ROT_WG_PER_CU 3
#define DSR_TUNE_ROT_GROUPED_WG_PER_CU 4
#define DSR_TUNE_SLOTS_TPW 5
#define DSR_TUNE_SLOTS_KERNEL 6
#define DSR_TUNE_SLOTS_UNROLL 7
#define DSR_TUNE_COPY_WG_PER_CU 8
#define DSR_TUNE_SCATTER_KERNEL 9
#define DSR_TUNE_GATHER_SPLIT 10
#define DSR_TUNE_PAGE_PARTS 11
#define DSR_TUNE_SLOTS_ORDER 12
#define DSR_TUNE_SLOTS_WG_PER_CU 13
#define DSR_TUNE_FANOUT_WG_PER_CU 14
#define DSR_TUNE_FANOUT_PARTS 15
#define DSR_TUNE_COUNT_ 16

#define DSR_OK 0
#define DSR_ERR_ARG (-1)   /* null pointer, negative count, bad enum     */
#define DSR_ERR_ALIGN (-2) /* a pointer/stride/size is not 16-byte aligned */
#define DSR_ERR_SHAPE (-3) /* rot_dim/head_dim/page geometry inconsistent */
#define DSR_ERR_IO (-4)    /* store-file read/write failed or came up short */
#define DSR_ERR_NOFILE (-5) /* store file does not exist                  */
#define DSR_ERR_TOO_LARGE (-6) /* tables exceed DSR_STATIC_TABLE_BYTES      */

/* Element types understood by the re-rotation kernel. Plain gather/scatter
 * is dtype-agnostic (raw bytes, bit-exact for every dtype incl. fp8). */
#define DSR_DTYPE_BF16 0
#define DSR_DTYPE_FP16 1
#define DSR_DTYPE_FP8_E4M3 2 /* OCP e4m3fn: bias 7, max 448, NaN 0x7F/0xFF */
#define DSR_DTYPE_FP8_E5M2 3 /* OCP e5m2: bias 15, max 57344, infinities, NaN */

/* RoPE pairings. */
#define DSR_ROPE_NEOX 0 /* rotate-half: pairs (j, j + rot_dim/2)  (Llama) */
#define DSR_ROPE_GPTJ 1 /* interleaved: pairs (2j, 2j + 1)                */

/* dsr_scatter_ex / dsr_scatter_rerotate* flags: several pages of the call
 * read the same records (a cached chunk placed in several requests). A
 * launch-shape hint; results do not depend on it. */
/* dsr_scatter_fanout cache page layouts. */
#define DSR_K_NHD 0 /* token-major [block_size][H][D]                         */
#define DSR_K_KX 1  /* split-x K [H][D / X][block_size][X] (3-D caches)       */
#define DSR_K_HND 2 /* head-major [H][block_size][D], records token-major     */

#define DSR_SHARED_RECORDS 1u
#define DSR_REROTATE_SHARED_RECORDS DSR_SHARED_RECORDS

/* Returns DSR_ABI_VERSION. */
int dsr_abi_version(void);

/* Human-readable text for a return code of this library. */
const char* dsr_error_string(int code);

/* Sets a launch-shape override (DSR_TUNE_*; 0 restores the default) for
 * every later call in this process. No counterpart in the reference: a
 * measurement and test hook, replacing per-call environment reads. Returns
 * DSR_ERR_ARG for an unknown knob or a negative value. */
int dsr_set_tuning(int knob, int64_t value);

/*
 * Offload gather: for every page p in [0, n_pages) and layer l in
 * [0, n_layers), copy the K and V pages of block page_ids[p] of layer l into
 * the slot record at staging + slot_offsets[p] + (layer0 + l) * layer_bytes.
 *
 * Replaces the per-(request, block) loop of DaserConnector.save_kv_layer,
 * reference daser/connector/daser_connector.py:610-632 (one launch covers
 * every store request of a step, and with n_layers > 1 every layer).
 *
 *   layer_base    [device] n_layers byte addresses of the per-layer caches
 *   kv_stride     bytes from a block's K page to its V page (kv.stride(0))
 *   page_stride   bytes between consecutive blocks (kv.stride(1))
 *   page_bytes    bytes of one K (or V) page
 *   num_blocks    blocks per layer cache (kv.shape[1])
 *   page_ids      [device] n_pages int32 block ids
 *   slot_offsets  [device] n_pages int64 offsets of each page's slot record
 *   staging       [device] destination records, staging_bytes long
 *   layer_bytes   record stride between layers (LAYER_SIZE)
 *   layer0        layer index of layer_base[0] inside the record
 */
int dsr_gather(const uint64_t* layer_base, int n_layers, int64_t kv_stride,
               int64_t page_stride, int64_t page_bytes, int64_t num_blocks,
               const int32_t* page_ids, const int64_t* slot_offsets,
               int n_pages, void* staging, int64_t staging_bytes,
               int64_t layer_bytes, int layer0, dsr_stream_t stream);

/*
 * Load scatter: the inverse of dsr_gather. Copies each slot record back into
 * the K and V pages of block page_ids[p] of every layer. A block may appear
 * once per call: pages are copied concurrently, so duplicates race (the
 * Python wrappers keep only the last entry of a block in host tables, the
 * bytes the reference's sequential copies leave). Listing pages in ascending block order makes
 * the writes near-sequential and is measurably faster.
 *
 * Replaces the per-(request, slot, layer) copy loop of
 * DaserConnector.start_load_kv, reference
 * daser/connector/daser_connector.py:536-551.
 */
int dsr_scatter(const uint64_t* layer_base, int n_layers, int64_t kv_stride,
                int64_t page_stride, int64_t page_bytes, int64_t num_blocks,
                const int32_t* page_ids, const int64_t* slot_offsets,
                int n_pages, const void* staging, int64_t staging_bytes,
                int64_t layer_bytes, int layer0, dsr_stream_t stream);

/* dsr_scatter with launch hints (flags: DSR_SHARED_RECORDS); the same
 * bytes. Same reference loop as dsr_scatter (daser_connector.py:536-551);
 * the hint is for loads in which requests share cached chunks. */
int dsr_scatter_ex(const uint64_t* layer_base, int n_layers, int64_t kv_stride,
                   int64_t page_stride, int64_t page_bytes, int64_t num_blocks,
                   const int32_t* page_ids, const int64_t* slot_offsets,
                   int n_pages, const void* staging, int64_t staging_bytes,
                   int64_t layer_bytes, int layer0, unsigned flags, dsr_stream_t stream);

/*
 * Load scatter with fused RoPE position-delta re-rotation of K.
 *
 * Same copy as dsr_scatter. In addition, for a page p with
 * rope_idx[p] >= 0, every K row (one token of one head, head_dim elements)
 * is rotated by the angle table cos_sin[rope_idx[p]][0 .. rot_dim/2):
 *   neox: (x_j, x_{j+R/2}) -> (x_j c_j - x_{j+R/2} s_j, x_{j+R/2} c_j + x_j s_j)
 *   gptj: (x_{2j}, x_{2j+1}) rotated the same way with (c_j, s_j)
 * with (c_j, s_j) = (cos, sin)(delta * inv_freq_j) and delta = new position
 * - stored position of the page's chunk, i.e. R(new) . R(stored)^-1 applied
 * in one step, fp32 arithmetic, one round to the storage type.
 * Elements j >= rot_dim and all V bytes are copied unchanged; pages with
 * rope_idx[p] < 0 are copied bit-exactly.
 *
 * fp8 (DSR_DTYPE_FP8_E4M3): x = e4m3(q) * k_scale[layer0 + l], rotate,
 * q' = e4m3_rne(clamp(y / k_scale, -448, 448)); NaN stays NaN (0x7F).
 * fp8 (DSR_DTYPE_FP8_E5M2): the same with e5m2 and +-57344; infinities
 * saturate too (a saturate-to-finite encode, the mode vLLM's fp8 cache
 * writes use, not torch's float8_e5m2 cast, which keeps infinities); NaN
 * -> 0x7F.
 * bf16/fp16: round-to-nearest-even from fp32; NaN -> canonical quiet NaN.
 *
 * The reference has no re-rotation (daser/position/fixed_offset.py:11-50
 * only carries an integer offset, which this path consumes); the copy it
 * fuses into replaces daser/connector/daser_connector.py:536-551.
 *
 * Models whose layers use different RoPE frequencies (e.g. local and global
 * attention layers with different bases) or no RoPE on some layers pass
 * layer_group: layer l of the record rotates with block layer_group[layer0 +
 * l] of the tables, and a layer with group -1 is copied unchanged.
 *
 *   cos_sin     [device] n_groups * n_tables * (rot_dim/2) float pairs
 *               (cos, sin): table t of group g at (g * n_tables + t)
 *   rope_idx    [device] n_pages int32 table index per page, -1 = no rotation
 *   n_tables    tables per group (bounds rope_idx)
 *   layer_group [device] int32 group of each record layer (indexed layer0 +
 *               l), -1 = no RoPE on that layer; null: one group for all
 *   n_groups    groups in cos_sin (>= 1 when layer_group is given)
 *   head_dim, rot_dim   rot_dim even, <= head_dim; head_dim * element size a
 *                       multiple of 16 bytes; page_bytes a multiple of one row
 *   k_scale   [device] per-layer fp32 scales, indexed layer0 + l; required
 *             for fp8, ignored otherwise (may be null). There is no V scale:
 *             V is copied as raw bytes, never decoded.
 *   flags     0, or DSR_REROTATE_SHARED_RECORDS when several pages of the
 *             call read the same records (one cached chunk placed in several
 *             requests): their repeated reads are served by the caches, and
 *             the launch is shaped for that (more workgroups per CU). A
 *             performance hint only: results are identical either way.
 */
int dsr_scatter_rerotate(const uint64_t* layer_base, int n_layers,
                         int64_t kv_stride, int64_t page_stride,
                         int64_t page_bytes, int64_t num_blocks,
                         const int32_t* page_ids, const int64_t* slot_offsets,
                         int n_pages, const void* staging,
                         int64_t staging_bytes, int64_t layer_bytes,
                         int layer0, const float* cos_sin,
                         const int32_t* rope_idx, int n_tables,
                         const int32_t* layer_group, int n_groups, int head_dim,
                         int rot_dim, int rope_style, int dtype,
                         const float* k_scale, unsigned flags, dsr_stream_t stream);

/*
 * Load of shared records: the bytes of dsr_scatter_rerotate (or, with
 * dst_rope_idx null, of dsr_scatter) for loads in which several pages read
 * the same record, with each record read once. Source s (record offset
 * src_offsets[s], layer l's part at + (layer0 + l) * layer_bytes) goes to
 * the destination blocks dst_page_ids[d] for d in [dst_start[s],
 * dst_start[s + 1]); destination d's K is rotated by table dst_rope_idx[d]
 * (-1: copied), exactly as dsr_scatter_rerotate rotates a page with that
 * table (same arithmetic, scales, layer groups and rounding). A block may
 * appear once per call (duplicates race). Out-of-range blocks and records
 * are skipped.
 *
 * The same loop of daser/connector/daser_connector.py:536-551 (each
 * request's pages copied from its staged chunk), for requests that share
 * cached chunks; the reference reads a shared chunk once per request.
 *
 * Geometry: pages of at most 32 KiB (8 vectors per lane); with rotation,
 * whole-vector rotary widths and neox partners a power of two <= 32 vectors
 * apart dividing the row, or gptj. k_layout names the cache pages:
 * DSR_K_NHD token-major (block_size and num_heads unused), DSR_K_KX the
 * split-x K pages of dsr_scatter_rerotate_kx (with its geometry conditions;
 * a plain copy moves them as raw bytes), DSR_K_HND head-major pages as for
 * the _hnd entry points (num_heads needed for a plain copy). Other shapes
 * return DSR_ERR_SHAPE (the per-page entry points cover them). The
 * geometry is checked before the tables: a call with n_src = n_dst = 0 and
 * null tables launches nothing and returns DSR_OK or DSR_ERR_SHAPE, whether
 * the fan-out takes these pages.
 *
 *   src_offsets   [device] n_src int64 record offsets
 *   dst_start     [device] n_src + 1 int32, non-decreasing, dst_start[0] = 0,
 *                 dst_start[n_src] = n_dst (trusted, as the tables' lengths
 *                 are: daser_amd.ops.fanout_tables builds it)
 *   dst_page_ids  [device] n_dst int32 block ids
 *   dst_rope_idx  [device] n_dst int32 table indices, or null (plain copy:
 *                 cos_sin, n_tables, layer_group, head_dim, rot_dim,
 *                 rope_style, dtype and k_scale are then ignored)
 */
int dsr_scatter_fanout(const uint64_t* layer_base, int n_layers, int64_t kv_stride,
                       int64_t page_stride, int64_t page_bytes, int64_t num_blocks,
                       const int64_t* src_offsets, int n_src, const int32_t* dst_start,
                       const int32_t* dst_page_ids, const int32_t* dst_rope_idx, int n_dst,
                       const void* staging, int64_t staging_bytes, int64_t layer_bytes,
                       int layer0, const float* cos_sin, int n_tables,
                       const int32_t* layer_group, int n_groups, int head_dim, int rot_dim,
                       int rope_style, int dtype, const float* k_scale, int k_layout,
                       int block_size, int num_heads, dsr_stream_t stream);

/*
 * Allocation-free form of dsr_scatter_rerotate. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (tight
 * serving loops, harnesses that forbid hipMalloc). Same arguments, kernels and bytes as dsr_scatter_rerotate,
 * except that layer_base, page_ids, slot_offsets, cos_sin, rope_idx,
 * layer_group and k_scale are HOST arrays: the call copies them
 * (hipMemcpyAsync on `stream`) into a fixed device array of the library
 * (DSR_STATIC_TABLE_BYTES per GPU, held until the process ends) and launches
 * on those copies. It calls no allocating routine.
 *
 * Limits and contracts:
 *   - the staged tables, each section rounded up to 256 bytes (layer_base 8 B
 *     per layer; page_ids 4, slot_offsets 8 and rope_idx 4 B per page;
 *     cos_sin n_groups * n_tables * rot_dim / 2 * 8 B; layer_group and
 *     k_scale 4 B per record layer), must fit in DSR_STATIC_TABLE_BYTES,
 *     else DSR_ERR_TOO_LARGE without any copy or launch (4 MiB holds e.g.
 *     130,000 pages of one layer group with 64 angle tables);
 *   - the host arrays must stay unchanged until `stream` has completed the
 *     call's work;
 *   - calls share the GPU's one array: calls on one stream are ordered, but
 *     calls that overlap on one GPU from different streams (or threads on
 *     different streams) race and must be serialised by the caller;
 *   - the device current on the calling thread must be the stream's device;
 *   - a stream under graph capture returns DSR_ERR_ARG (the host-to-device
 *     table copies cannot be captured).
 */
#define DSR_STATIC_TABLE_BYTES (4 << 20)
int dsr_scatter_rerotate_static(const uint64_t* layer_base, int n_layers,
                                int64_t kv_stride, int64_t page_stride,
                                int64_t page_bytes, int64_t num_blocks,
                                const int32_t* page_ids, const int64_t* slot_offsets,
                                int n_pages, const void* staging,
                                int64_t staging_bytes, int64_t layer_bytes,
                                int layer0, const float* cos_sin,
                                const int32_t* rope_idx, int n_tables,
                                const int32_t* layer_group, int n_groups, int head_dim,
                                int rot_dim, int rope_style, int dtype,
                                const float* k_scale, unsigned flags, dsr_stream_t stream);

/*
 * dsr_scatter_rerotate for caches whose K page uses the split-x layout of
 * vLLM's PagedAttention kernels (its ROCm paged-attention backend: caches of
 * shape (2, num_blocks, block_size * H * D), K viewed as
 * [H][D / X][block_size][X] with X = 16 / element bytes, V as
 * [H][D][block_size]). Element (token t, head h, dim d) of K sits at element
 *     ((h * (D / X) + d / X) * block_size + t) * X + d % X
 * of the page. The rotation is the same as dsr_scatter_rerotate's, per
 * (t, h) over dims d < rot_dim; V and unrotated pages are copied bit-exactly
 * (the copy entry points need no layout: they move whole pages).
 *
 * Replaces the same reference loop as dsr_scatter_rerotate
 * (daser/connector/daser_connector.py:536-551, whose per-page copy_ moves
 * kv[:, b] of any cache shape). Extra constraints: block_size > 0; page_bytes
 * a multiple of block_size * head_dim * elem_bytes; rot_dim / 2 (neox) or
 * rot_dim (gptj) a multiple of X; head_dim - rot_dim a multiple of X.
 */
int dsr_scatter_rerotate_kx(const uint64_t* layer_base, int n_layers,
                            int64_t kv_stride, int64_t page_stride,
                            int64_t page_bytes, int64_t num_blocks,
                            const int32_t* page_ids, const int64_t* slot_offsets,
                            int n_pages, const void* staging,
                            int64_t staging_bytes, int64_t layer_bytes,
                            int layer0, const float* cos_sin,
                            const int32_t* rope_idx, int n_tables,
                            const int32_t* layer_group, int n_groups, int head_dim,
                            int rot_dim, int rope_style, int dtype,
                            const float* k_scale, int block_size, unsigned flags,
                            dsr_stream_t stream);

/*
 * Head-major cache pages: vLLM's optional HND KV layout keeps the caches'
 * logical shape (2, num_blocks, block_size, H, D) but stores a page with its
 * heads outermost, [H][block_size][D]. The record of a page is still
 * bytes(kv_l[:, b]) in logical, token-major order [block_size][H][D] (the
 * reference's reshape(-1), daser/connector/daser_connector.py:625-632, and
 * its copy_ back, :545-550), so these entry points permute whole rows of D
 * elements between the two orders: row (t, h) of the record is row
 * h * block_size + t of the cache page. Same arguments and contracts as
 * dsr_gather / dsr_scatter / dsr_scatter_rerotate, plus the page geometry:
 * block_size and num_heads with page_bytes a multiple of block_size *
 * num_heads * 16 (the copies); block_size, with page_bytes a multiple of
 * block_size * head_dim * elem_bytes (the re-rotation, whose rotary widths
 * must be whole 16-byte vectors with a power-of-two neox partner distance
 * of at most 32 vectors, or gptj; other shapes return DSR_ERR_SHAPE).
 */
int dsr_gather_hnd(const uint64_t* layer_base, int n_layers, int64_t kv_stride,
                   int64_t page_stride, int64_t page_bytes, int64_t num_blocks,
                   const int32_t* page_ids, const int64_t* slot_offsets, int n_pages,
                   void* staging, int64_t staging_bytes, int64_t layer_bytes, int layer0,
                   int block_size, int num_heads, dsr_stream_t stream);

int dsr_scatter_hnd(const uint64_t* layer_base, int n_layers, int64_t kv_stride,
                    int64_t page_stride, int64_t page_bytes, int64_t num_blocks,
                    const int32_t* page_ids, const int64_t* slot_offsets, int n_pages,
                    const void* staging, int64_t staging_bytes, int64_t layer_bytes,
                    int layer0, int block_size, int num_heads, dsr_stream_t stream);

int dsr_scatter_rerotate_hnd(const uint64_t* layer_base, int n_layers,
                             int64_t kv_stride, int64_t page_stride,
                             int64_t page_bytes, int64_t num_blocks,
                             const int32_t* page_ids, const int64_t* slot_offsets,
                             int n_pages, const void* staging,
                             int64_t staging_bytes, int64_t layer_bytes,
                             int layer0, const float* cos_sin,
                             const int32_t* rope_idx, int n_tables,
                             const int32_t* layer_group, int n_groups, int head_dim,
                             int rot_dim, int rope_style, int dtype,
                             const float* k_scale, int block_size, unsigned flags,
                             dsr_stream_t stream);

/*
 * Token-granular offload gather driven by vLLM's slot_mapping: for every
 * token t in [0, n_tokens) with slot = slot_mapping[t] >= 0 and every layer
 * l, copy its K row (all heads: row_bytes = H * D * elem_bytes) from
 *     layer_base[l] + (slot / block_size) * page_stride
 *                   + (slot % block_size) * row_bytes
 * to  staging + row_offsets[t] + (layer0 + l) * layer_bytes,
 * and its V row (+ kv_stride in the cache) to the same place + page_bytes.
 * Tokens with slot < 0 (vLLM's padding) are skipped. With row_offsets[t] =
 * record(t / block_size) + (t % block_size) * row_bytes this writes exactly
 * the slot records of dsr_gather, restricted to the valid tokens (a partial
 * last page leaves its tail rows untouched).
 *
 * Per-token form of the save loop of daser/connector/daser_connector.py:
 * 625-632 (which copies whole pages, :280); slot = block_ids[t / bs] * bs +
 * t % bs is vLLM's slot_mapping for the same tokens.
 *
 *   slot_mapping  [device] n_tokens int64 slots (block * block_size + offset)
 *   row_offsets   [device] n_tokens int64 record offsets of each token's K row
 */
int dsr_gather_slots(const uint64_t* layer_base, int n_layers, int64_t kv_stride,
                     int64_t page_stride, int64_t page_bytes, int64_t num_blocks,
                     int block_size, int64_t row_bytes, const int64_t* slot_mapping,
                     const int64_t* row_offsets, int n_tokens, void* staging,
                     int64_t staging_bytes, int64_t layer_bytes, int layer0,
                     dsr_stream_t stream);

/*
 * Inverse of dsr_gather_slots: each valid token's K and V rows are copied
 * from its record rows back to slot slot_mapping[t] of every layer. Per-token
 * form of the load loop of daser/connector/daser_connector.py:536-551.
 */
int dsr_scatter_slots(const uint64_t* layer_base, int n_layers, int64_t kv_stride,
                      int64_t page_stride, int64_t page_bytes, int64_t num_blocks,
                      int block_size, int64_t row_bytes, const int64_t* slot_mapping,
                      const int64_t* row_offsets, int n_tokens, const void* staging,
                      int64_t staging_bytes, int64_t layer_bytes, int layer0,
                      dsr_stream_t stream);

/*
 * Token-form load with the fused re-rotation: dsr_scatter_slots, and the K
 * row of each valid token t with rope_idx[t] >= 0 has every head's first
 * rot_dim dims rotated by the table cos_sin[rope_idx[t]] exactly as
 * dsr_scatter_rerotate rotates a page row (same pairs, scales, rounding,
 * layer groups). Heads must be a power-of-two number of 16-byte vectors
 * (<= 64), rot_dim <= 256 in whole vectors (each half, for neox); else
 * DSR_ERR_SHAPE. Per-token form of the load loop of
 * daser/connector/daser_connector.py:536-551 plus the re-rotation, which
 * the reference does not have.
 */
int dsr_scatter_slots_rerotate(const uint64_t* layer_base, int n_layers, int64_t kv_stride,
                               int64_t page_stride, int64_t page_bytes, int64_t num_blocks,
                               int block_size, int64_t row_bytes, const int64_t* slot_mapping,
                               const int64_t* row_offsets, int n_tokens, const void* staging,
                               int64_t staging_bytes, int64_t layer_bytes, int layer0,
                               const float* cos_sin, const int32_t* rope_idx, int n_tables,
                               const int32_t* layer_group, int n_groups, int head_dim,
                               int rot_dim, int rope_style, int dtype, const float* k_scale,
                               dsr_stream_t stream);

/*
 * Pinned-host staging ring between device records and the store file.
 *
 * Replaces the reference's kvikio layer, daser/connector/gds_transfer.py:
 * 22-127 (GDSTransferLayer: __init__ opens an existing store file and raises
 * FileNotFoundError otherwise, :49-50; write_async / read_into_async move a
 * GPU buffer to / from a file offset, :72-116; close, :118-121).
 *
 * A transfer of n bytes is cut into slot_bytes pieces that cycle through
 * n_slots pinned host buffers: device <-> slot copies run as
 * hipMemcpyAsync on a ring-owned stream, file I/O as io_uring READ/WRITE
 * submitted from the calling thread (pread/pwrite when io_uring is
 * unavailable). Pieces overlap: while piece k is written, piece k+1 is
 * being copied. Calls on one ring serialise on an internal mutex.
 */
typedef struct dsr_ring dsr_ring;

#define DSR_RING_HOST 1     /* src/dst are host memory: memcpy, no HIP calls */
#define DSR_RING_DIRECT 2   /* open the file with O_DIRECT: slot_bytes, file
                               offsets and transfer sizes must be multiples of
                               4096 (DSR_ERR_ALIGN otherwise). The slots are
                               then 4 KiB-aligned pageable memory (O_DIRECT
                               cannot use hipHostMalloc'd pages)            */
#define DSR_RING_NO_URING 4 /* use pread/pwrite even if io_uring works       */
#define DSR_RING_MMAP 8     /* copy between the pinned slots and a shared
                               mapping of the file on worker threads (up to
                               8, one per slot) instead of read/write calls:
                               buffered writes to one file serialise in the
                               kernel, page faults on a mapping do not. A
                               write first allocates the blocks of its range
                               (fallocate: ENOSPC is DSR_ERR_IO, not a fault);
                               a write past the end of the file goes through
                               pwrite/io_uring.
                               Not with DSR_RING_DIRECT (DSR_ERR_ARG). The
                               file must not be truncated while the ring is
                               open (a mapped access past its end faults)  */

/* Opens `path` (must exist: DSR_ERR_NOFILE otherwise) and allocates the
 * ring. slot_bytes <= 2^31 - 1, 1 <= n_slots <= 65535. */
int dsr_ring_open(const char* path, int64_t slot_bytes, int n_slots, int flags,
                  dsr_ring** out);

/* Writes nbytes of `src` (device memory unless DSR_RING_HOST) at
 * file_offset. Work enqueued on `producer` before the call is complete
 * before the copy. Returns when every byte has been written to the file
 * (or an error: DSR_ERR_IO, errno in dsr_ring_last_errno). */
int dsr_ring_write(dsr_ring* ring, const void* src, int64_t nbytes, int64_t file_offset,
                   dsr_stream_t producer);

/* Reads nbytes at file_offset into `dst`. Work enqueued on `consumer` before
 * the call (which may still use dst) is complete before the first copy into
 * dst; on return the file reads are done and `consumer` is ordered after the
 * last copy. A read past the end of the file is DSR_ERR_IO. */
int dsr_ring_read(dsr_ring* ring, void* dst, int64_t nbytes, int64_t file_offset,
                  dsr_stream_t consumer);

/* 1 if transfers go through io_uring, 0 if through pread/pwrite. */
int dsr_ring_uses_io_uring(const dsr_ring* ring);

/* 1 if the ring was opened with DSR_RING_MMAP. No counterpart in the
 * reference (its GDSTransferLayer.backend names kvikio's mode). */
int dsr_ring_is_mapped(const dsr_ring* ring);

/* errno of the last failed file operation on this ring (0 if none). */
int dsr_ring_last_errno(const dsr_ring* ring);

/* Waits for the ring's copies, frees its buffers and closes the file. */
int dsr_ring_close(dsr_ring* ring);

#ifdef __cplusplus
}
#endif

#endif /* DASER_KV_H */
