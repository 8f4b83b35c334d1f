/*
 * spconv_amd -- C ABI of the MI355X (gfx950) submanifold sparse-convolution path.
 *
 * This is the drop-in boundary for the reference's sparse-conv entry points (suvadityamuk/trellis2-cuda
 * src/spconv.h:5-16) exported the way the reference exports its pipeline to ctypes (apps/t2lib.cu:1-23):
 * every call returns 0 on success or -1 with spc_last_error() set; calls are serialized by one mutex.
 * All data pointers are DEVICE pointers (HIP, the library's current device) unless marked "host".
 * Work is ordered on one stream (default: the null stream; see spc_set_stream).
 *
 * dtype codes follow the reference's DT enum (src/core.h:22): 0 = fp32, 1 = fp16, 2 = bf16.
 */
#ifndef SPCONV_AMD_H
#define SPCONV_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { SPC_F32 = 0, SPC_F16 = 1, SPC_BF16 = 2 };
enum { SPC_ACT_NONE = 0, SPC_ACT_SILU = 1 };
/* Or'ed into a conv's act: the reference's fp16 rounding sequence instead of one rounding -- y = f16(f16(acc) + b),
 * then y = f16(y / (1 + exp(-y))) for SiLU, then y = f16(y + residual) (src/spconv.cu:141-143, src/ops.cu:79-82,
 * 105-113). x, w, out fp16; bias and residual fp16 or NULL. */
enum { SPC_EPI_F16_COMPAT = 256 };
#define SPC_EMPTY 0xffffffffu

typedef struct spc_cache spc_cache; /* owns one SpConvCache (reference src/spconv.h:6-11) */

/* Last error message of the calling process (reference apps/t2lib.cu:23 t2_last_error). */
const char* spc_last_error(void);

/* Make `hip_stream` (a hipStream_t, or NULL for the null stream) the stream every later call runs on.
 * Reference: the single global stream of src/core.cu:20-28. */
int spc_set_stream(void* hip_stream);

/* Build the hash table and 27-offset neighbour map of `coords` (int32 [n,4] = (b,x,y,z), unique rows) in a
 * W x H x D grid, plus the gray-code sorted row order.
 * Replaces: build_neighbors (src/spconv.h:12, src/spconv.cu:38-54). */
int spc_build_neighbors(const int32_t* coords, int64_t n, int W, int H, int D, spc_cache** out);

/* As spc_build_neighbors, with flags: SPC_KEEP_HASH keeps the voxel hash in the cache (about 32-128 + 256 bytes
 * per voxel) for spc_cache_lookup.
 * Replaces: build_neighbors (src/spconv.cu:38-54) and the voxel hash builds of other consumers (k_vhash_insert,
 * src/mesh.cu:8-13; the bake's hash, src/glb.cu:548-550), which can query this one instead. */
enum { SPC_KEEP_HASH = 1 };
int spc_build_neighbors_ex(const int32_t* coords, int64_t n, int W, int H, int D, int flags, spc_cache** out);

/* rows[i] = the row of query[i] (int32 [m,4] = (b,x,y,z)) in the cache's voxels, or -1 when absent or outside the
 * grid. Needs a cache built with SPC_KEEP_HASH (an empty cache answers -1).
 * Replaces: vhash_find (src/mesh.cu:14-19) and the reference's per-offset probes (src/spconv.cu:22-36). */
int spc_cache_lookup(const spc_cache* c, const int32_t* query, int64_t m, int32_t* rows);

/* FlexiDualGrid quads from the cache's kernel map, no hash probes: for e = 3i + a, ok[e] = 1 and quad[e] = the rows
 * of the 4 voxels at axis a's edge offsets when h[i, 3+a] > 0 (h f32 [n,7]) and all 4 exist, else ok[e] = 0 and
 * quad[e] is left untouched. quad int32 [3n,4] (16-byte aligned), ok int32 [3n]. Matches the reference for a cache
 * built over one batch with W = H = D = R.
 * Replaces: k_fdg_quads and its hash (src/mesh.cu:7-19, 36-45, 54-62). */
int spc_fdg_quads(const spc_cache* c, const float* h, int32_t* quad, int32_t* ok);

/* Trilinear sample map of L points grid f32 [L,3] (continuous voxel coordinates: voxel i spans [i, i+1)) in batch
 * `batch` of a cache built with SPC_KEEP_HASH: nb u32 [L,8] = the rows of the 8 voxels around p - 0.5 (corner
 * v = dx*4 + dy*2 + dz; SPC_EMPTY when absent or off-grid), wt f32 [L,8] = their trilinear weights (0 for EMPTY
 * corners). flags: SPC_GS_NORMALIZE divides the present weights by their sum.
 * Replaces: the bake's FlexGEMM hashmap_build_grid_sample_3d_trilinear_neighbor_map_weight and its voxel hash
 * (src/glb.cu:547-550). */
enum { SPC_GS_NORMALIZE = 1 };
int spc_grid_sample_map(const spc_cache* c, const float* grid, int64_t L, int batch, int flags, uint32_t* nb,
                        float* wt);

/* y f32 [L,C] = sum over v of x[nb[i,v]] * wt[i,v] (x f32 [M,C]; fused multiply-adds in v order, SPC_EMPTY reads 0).
 * Replaces: k_wsum (src/glb.cu:456-465, launched at :552). */
int spc_grid_sample_sum(const float* x, int64_t M, int C, const uint32_t* nb, const float* wt, int64_t L, float* y);

/* Release a cache (its device buffers are freed in stream order). */
int spc_cache_free(spc_cache* c);

/* Device pointers owned by the cache: nbr u32 [n,27] (SPC_EMPTY = none), gray i32 [n] (27-bit mask),
 * sorted i32 [n]. Any out-pointer may be NULL. Replaces the fields of SpConvCache (src/spconv.h:7-8). */
int spc_cache_info(const spc_cache* c, int64_t* n, const uint32_t** nbr, const int32_t** gray,
                   const int32_t** sorted);

/* Per-block valid offset lists for blocks of B1 sorted rows: list (device, worst-case length 27*ceil(n/B1)),
 * seg (device, ceil(n/B1)+1 entries, list[seg[b]:seg[b+1]] ascending). If L (host) is non-NULL the call waits
 * for the stream and stores seg[last] there. Memoized per B1.
 * Replaces: SpConvCache::valid (src/spconv.h:10, src/spconv.cu:56-75). */
int spc_cache_valid(spc_cache* c, int B1, const int32_t** list, const int32_t** seg, int64_t* L);

/* Tile choice for an (N, Ci, Co) conv: rows per tile/schedule block B1, channels per K stage BK, split S.
 * Replaces: spconv_cfg (src/spconv.h:13-14, src/spconv.cu:177-221); the tile table is fixed per width. */
int spc_conv_cfg(int64_t N, int Ci, int Co, int* B1, int* BK, int* S);

/* The reference's tile choice replayed from a FlexGEMM autotune cache file (`path`, device section `device`, e.g.
 * "NVIDIA H200"): split S from the splitk table, then B1/BK for (floor(log2 N), Ci, Co, S); 128/64/1 where the file
 * has no entry. Host only (no GPU needed); the file is parsed once per (path, device). This build's kernels keep their
 * own tiles; B1 here gives the reference's schedule blocks for spc_cache_valid.
 * Replaces: spconv_cfg's table replay (src/spconv.cu:176-221). */
int spc_conv_cfg_autotune(const char* path, const char* device, int64_t N, int Ci, int Co, int* B1, int* BK, int* S);

/* spc_conv_cfg_autotune with strict replay: when `strict` is nonzero (or the environment has T2_STRICT=1, which
 * spc_conv_cfg_autotune honours too) a (N, Ci, Co) the file has no tile entry for is an error (-1 and
 * spc_last_error) instead of the 128/64 default, so a replayed tile cannot be mistaken for a default one.
 * Replaces: spconv_cfg's strict mode (src/spconv.cu:219). */
int spc_conv_cfg_autotune_strict(const char* path, const char* device, int64_t N, int Ci, int Co, int strict, int* B1,
                                 int* BK, int* S);

/* out[N,Co] (dtype = x's) = subm_conv3d(x [N,Ci], w [Co,27,Ci], b [Co] or NULL).
 * x and w: both SPC_F16 or both SPC_BF16; b_dtype: SPC_F32/F16/BF16. Ci % 32 == 0, Co % 64 == 0.
 * Replaces: subm_conv (src/spconv.h:15-16, src/spconv.cu:159-175); the output buffer is the caller's. */
int spc_subm_conv(const void* x, const void* w, const void* b, int dtype, int b_dtype, int64_t N, int Ci, int Co,
                  spc_cache* c, void* out);

/* Fused epilogue variant: out = act(conv(x) + b) [+ residual], one rounding to out_dtype (F32/F16/BF16);
 * residual [N,Co] of res_dtype or NULL; act = SPC_ACT_NONE / SPC_ACT_SILU (silu(v) = v / (1 + exp(-v))).
 * Replaces: subm_conv followed by the separate act_/add_ passes of src/ops.cu:79-82,105-113 (no reference
 * entry point fuses them). */
int spc_subm_conv_fused(const void* x, const void* w, const void* b, const void* residual, int dtype, int b_dtype,
                        int res_dtype, int out_dtype, int act, int64_t N, int Ci, int Co, spc_cache* c, void* out);

/* Conv of gathered rows: as spc_subm_conv_fused with x = x_src[row_map[i] >> shift] (x_src [M,Ci], row_map int32
 * [N], N = the cache's rows; map entries outside [0,M) read zero rows), without materializing the gathered rows.
 * With the c2s outputs (row_map = src, shift = 3) this is a decoder upsample block's gather + conv.
 * Replaces: SDecoder's k_gather_rows followed by subm_conv (src/sdec.cu:34-43, 70-87). */
int spc_subm_conv_gathered(const void* x_src, int64_t M, const int32_t* row_map, int shift, const void* w,
                           const void* b, const void* residual, int dtype, int b_dtype, int res_dtype, int out_dtype,
                           int act, int64_t N, int Ci, int Co, spc_cache* c, void* out);

/* Pre-activation in one pass: out[i] = act(LayerNorm(x_src[row_map[i] >> shift]) * gamma + beta), statistics in
 * fp32, one rounding; x_src [M,C] and out [N,C] both `dtype` (SPC_F16/SPC_BF16), gamma/beta f32 [C] or NULL,
 * act SPC_ACT_NONE/SPC_ACT_SILU, C = 8 * 2^k <= 4096. Map entries outside [0,M) read zero rows (out = act(beta));
 * row_map NULL is the identity (N = M).
 * Replaces: layer_norm + act_(SILU) (src/ops.cu:30-75, src/sdec.cu:72-73) and, with row_map = the c2s src and
 * shift = 3, k_gather_rows + layer_norm + act_ (src/sdec.cu:34-43, 78-83). */
int spc_gather_ln_act(const void* x_src, int64_t M, int C, const int32_t* row_map, int shift, const float* gamma,
                      const float* beta, float eps, int act, int dtype, int64_t N, void* out);

/* ConvNeXt tail in one pass: y = x + W2 silu(W1 (LayerNorm(h) * gamma + beta) + b1) + b2 per row, fp32 statistics
 * and accumulation, the hidden activations rounded to `dtype` between the two products, one rounding of y.
 * h, x, y [N,C], w1 [4C,C], w2 [C,4C] (torch Linear layout): `dtype` (SPC_F16/SPC_BF16), 16-byte aligned;
 * gamma, beta, b2 [C] and b1 [4C]: `param_dtype` or NULL (gamma 1, others 0); C = 64, 128 or 256 (one fused pass)
 * or 512, 1024 (LayerNorm pass, then two GEMM passes with the bias/SiLU and bias/residual epilogues).
 * y may alias h or x.
 * Replaces: the tail of SDecoder::convnext after its conv -- layer_norm, linear, act_ SILU, linear, add_
 * (src/sdec.cu:60-66, src/ops.cu:30-75, src/gemm.cu:24-63). */
int spc_convnext_mlp(const void* h, const void* x, const void* gamma, const void* beta, float eps, const void* w1,
                     const void* b1, const void* w2, const void* b2, int dtype, int param_dtype, int64_t N, int C,
                     void* y);

/* Conv and the upsample block's skip connection in one pass: out = act(conv(x, w) + b) + skip with skip[i,c] =
 * x_skip[src[i] >> 3, (src[i] & 7) * Cin/8 + c / rep], rep = Co / (Cin/8) a power of two; fp32 sum, one rounding.
 * x [N,Ci], w [Co,27,Ci], x_skip [n_skip,Cin] (Cin % 64 == 0), out [N,Co]: one 16-bit `dtype`; src int32 [N] (the
 * c2s output). Fused into the 64 -> 64 kernel; other shapes run the conv and spc_add_skip's pass.
 * Replaces: subm_conv + k_add_skip of SDecoder::up (src/sdec.cu:38-43, 82-84). */
int spc_subm_conv_skip(const void* x, const void* w, const void* b, int dtype, int b_dtype, int act,
                       const void* x_skip, int64_t n_skip, int Cin, const int32_t* src, int64_t N, int Ci, int Co,
                       spc_cache* c, void* out);

/* Conv of pre-activated rows: x = pre_act(LayerNorm(x_src[row_map[i] >> shift]) * gamma + beta) (fp32 statistics,
 * one rounding; row_map NULL: the rows of x_src, M == N), out = act(conv(x, w) + b), plus, when x_skip / skip_src
 * are given, the skip of spc_subm_conv_skip. x_src [M,Ci], w [Co,27,Ci], x_skip [n_skip,Cin], out [N,Co]: one
 * 16-bit `dtype`; gamma, beta float [Ci] or NULL; pre_act SPC_ACT_NONE / SPC_ACT_SILU. Runs spc_gather_ln_act's
 * pass and then the conv; with the environment switch SPCONV_PRELN_FUSED=1, 64 -> 64 convs whose schedule has no
 * spill tiles run as one kernel (the pre-activation applied to each tile's distinct input rows in LDS; slower on
 * the shapes measured) -- the same bits either way.
 * Replaces: k_gather_rows + layer_norm + act_ SILU + subm_conv (+ k_add_skip) of SDecoder::up (src/sdec.cu:78-84,
 * src/ops.cu:30-82). */
int spc_subm_conv_preln(const void* x_src, int64_t M, const int32_t* row_map, int shift, const float* gamma,
                        const float* beta, float eps, int pre_act, const void* w, const void* b, int dtype, int b_dtype,
                        int act, const void* x_skip, int64_t n_skip, int Cin, const int32_t* skip_src, int64_t N,
                        int Ci, int Co, spc_cache* c, void* out);

/* Skip connection of the upsample block, in place: h[i,c] += x[src[i] >> 3, (src[i] & 7) * Cin/8 + c / rep] with
 * rep = Co / (Cin/8), the fp32 sum rounded once to `dtype` (bit-identical to the reference); h [m,Co], x [n,Cin],
 * both SPC_F16 or SPC_BF16, 16-byte aligned; Cin % 8 == 0, Co % 8 == 0, Co % (Cin/8) == 0. src entries outside
 * [0, 8n) leave their row unchanged.
 * Replaces: k_add_skip (src/sdec.cu:38-43, launched at :84). */
int spc_add_skip(void* h, const void* x, const int32_t* src, int64_t m, int Co, int64_t n, int Cin, int dtype);

/* The reference's fp16 conv under a given tile choice (B1, BK, S) -- e.g. spc_conv_cfg_autotune's -- rounding
 * included: S == 1 is spc_subm_conv_fused with SPC_EPI_F16_COMPAT; S > 1 computes fp32 partials per split (each split
 * takes its share of every B1-row block's K chunks, the fp32 bias goes into split 0) and sums them with four
 * interleaved accumulators before one fp16 rounding; act (SPC_ACT_NONE/SPC_ACT_SILU) and residual (or NULL) then
 * round as the reference's separate passes. x, w, b, residual, out: fp16. B1 and BK multiples of 32, Ci % BK == 0,
 * Co % 32 == 0, 1 <= S <= 64.
 * Replaces: subm_conv's k_spconv + k_splitk_sum path and its act_ / add_ passes (src/spconv.cu:90-175,
 * src/ops.cu:79-82,105-113). */
int spc_subm_conv_replay(const void* x, const void* w, const void* b, const void* residual, int act, int64_t N, int Ci,
                         int Co, int B1, int BK, int S, spc_cache* c, void* out);

/* Child subdivision (c2s): children of each parent whose fp16 logit (logits [n,8]) is > 0, in (parent, slot)
 * order; child_coords int32 [>= 8n, 4] and src int32 [>= 8n] receive the children, *m (host) their count
 * (the call waits for the stream, as the reference does at src/sdec.cu:52).
 * Replaces: SDecoder::c2s's k_c2s_count / scan / k_c2s_emit (src/sdec.cu:20-33,45-54). */
int spc_subdivide(const int32_t* coords, const uint16_t* logits_f16, int64_t n, int32_t* child_coords,
                  int32_t* src, int64_t* m);

/* Subdivision and the children's kernel map in one call, with no host sync between them: children into
 * child_coords int32 [>= 8n, 4] and src int32 [>= 8n] as spc_subdivide, *m (host) their count, *out a cache equal
 * to spc_build_neighbors(child_coords, *m, W, H, D). The map build is launched for the 8n capacity and stops at the
 * count on the device; the count is copied back while the build runs.
 * Replaces: SDecoder::c2s -- k_c2s_count / scan / host read of the count / k_c2s_emit, then build_neighbors on the
 * children (src/sdec.cu:45-56). */
int spc_subdivide_build(const int32_t* coords, const uint16_t* logits_f16, int64_t n, int W, int H, int D,
                        int32_t* child_coords, int32_t* src, int64_t* m, spc_cache** out);

/* spc_subdivide without allocating and without waiting: the same children into child_coords int32 [>= 8n, 4] and
 * src int32 [>= 8n], their count into *m_dev (DEVICE int64). No counterpart in the reference: it is for callers that
 * cannot allocate device memory or block on the host (code under HIP graph capture, tight serving loops). Its
 * scratch (per-parent counts and scan sums, about 16 MiB) is a static device array that each GPU holds until the
 * process ends, so n <= 4194304 (larger n fails with an error) and calls that overlap on one GPU race. */
/* Conv-kernel timing. spc_kernel_timing(1) clears the list and starts bracketing each conv call's conv kernels (split-K
 * reduction and spill-tile kernel included; weight repack and first-call schedules excluded) with HIP events on the
 * library stream; spc_kernel_timing(0) stops. spc_kernel_times waits for the recorded events and writes up to `max`
 * per-call kernel times (ms, call order) to ms, their number to *n. No counterpart in the reference (its parity app
 * times whole calls, apps/parity.cu:148-167): it separates the kernels from the per-call weight repack. */
int spc_kernel_timing(int on);
int spc_kernel_times(float* ms, int max, int* n);

/* Device allocations the library has made in this process: *requests counts every nonzero-sized allocation request
 * (served from its free lists or not), *driver_allocs the hipMallocAsync calls among them. No counterpart in the
 * reference: a diagnostic for callers that must not allocate (compare the counts around a call). Host only. */
int spc_alloc_counts(int64_t* requests, int64_t* driver_allocs);

/* Returns the library's cached, currently unused device blocks to the driver (the library keeps freed blocks for
 * reuse, as a framework's caching allocator does) and trims the device memory pools; waits for the devices those
 * blocks belong to. *bytes (may be NULL) receives the bytes released. Blocks held by live caches are untouched.
 * Replaces: nothing in the reference, whose allocator frees on release (src/core.cu:32-40); for pipelines that run
 * other large models between decoder passes. */
int spc_release_cached_memory(int64_t* bytes);

int spc_subdivide_noalloc(const int32_t* coords, const uint16_t* logits_f16, int64_t n, int32_t* child_coords,
                          int32_t* src, int64_t* m_dev);

#ifdef __cplusplus
}
#endif
#endif
