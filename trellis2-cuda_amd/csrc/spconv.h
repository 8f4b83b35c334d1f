// Submanifold 3x3x3 sparse convolution on MI355X: the C++ API of the reference's src/spconv.h:1-16, kept
// call-compatible so the sparse decoders (reference src/sdec.cu:15-18, 55, 92) can call it unchanged.
#pragma once
#include <map>
#include <vector>
#include <utility>

#include "core.h"

// The C++ API is exported from libspconv_amd.so (the library builds with hidden visibility otherwise), so C++
// callers such as the sparse decoders link against it directly.
#pragma GCC visibility push(default)

// Neighbour cache for one coordinate set (reference src/spconv.h:5-11).
//   nbr    [N,27] u32, 0xffffffff = no neighbour, offset v <-> (dx,dy,dz) = (v/9-1, v/3%3-1, v%3-1)
//   gray   [N] i32   27-bit neighbour mask
//   sorted [N] i32   stable ascending order of the gray-decoded mask (ties keep row order)
//   vk     B1 -> (valid offset list, segment offsets [ceil(N/B1)+1]); list is allocated at its worst case
//          27*ceil(N/B1) (no host sync); its used length is seg[ceil(N/B1)].
struct SpConvCache {
  int N = 0;
  Tensor nbr, gray, sorted;
  std::map<int, std::pair<Tensor, Tensor>> vk;
  const std::pair<Tensor, Tensor>& valid(int B1);
  // Per-block OR of the neighbour masks over B1 consecutive sorted rows: the conv kernel's schedule. The set
  // bits of masks[b] are exactly list[seg[b]:seg[b+1]].
  std::map<int, Tensor> masks;
  const Tensor& block_masks(int B1);
  // Rows grouped by spatial window (row >> log2w, i.e. runs of 2^log2w rows of the input order) and, inside a
  // window, in the gray-sorted order: neighbour masks stay similar within small row groups while the rows a tile
  // gathers stay spatially close. Used by the narrow-channel kernels.
  std::map<int, Tensor> worder;
  const Tensor& window_order(int log2w);
  // The neighbour table in a tile order, so a conv tile reads its rows' neighbour indices as one contiguous block:
  // tbl[i] = nbr[order[i]] (27 u32, EMPTY kept) and gs[i] = gray[order[i]], padded with EMPTY rows and zero masks
  // to a multiple of kRowTablePad rows; order = window_order(log2w), or sorted for log2w < 0. Memoized, like the
  // schedules above: a decoder runs many convs on one cache.
  static constexpr int kRowTablePad = 256;
  struct RowTable {
    Tensor order, tbl, gs;
  };
  std::map<int, RowTable> rtab;
  const RowTable& row_table(int log2w);
  // Tiles of B consecutive entries of row_table(log2w) in dispatch order: longest first (by the number of offsets
  // in the tile's union mask, the tile's K stages), so the last workgroups of a launch are the short ones.
  // Memoized per (log2w, B).
  std::map<std::pair<int, int>, Tensor> tsched;
  const Tensor& tile_schedule(int log2w, int B);
  // row_table(log2w).tbl with every non-EMPTY entry r replaced by row_map[r] >> shift, or EMPTY when that is not
  // below m (not memoized: row_map is the caller's). Used by the gathered conv.
  Tensor mapped_table(int log2w, const Tensor& row_map, int shift, i64 m);
  // Halo schedule for the 64-output-channel convs: tiles of B consecutive rows of the input order, gray-sorted inside
  // (order). Per tile: the distinct neighbour rows it reads (rows[t*UM + u], u < count[t]), each position's 27
  // neighbours as indices into that list (idx[(t*27 + v)*B + j], u16; UM = EMPTY, a zero row) and the per-16-position
  // neighbour masks (gm[t*B/16 + g]). A tile that reads more than UM distinct rows is a spill tile: count[t] = -1 (the
  // halo kernel skips it) and its index is in spill_list (spill_count entries, on the device; the gathering kernel
  // computes those tiles). Built on first use per (B, UM) in one launch with no host sync, memoized.
  struct HaloTable {
    Tensor order, rows, count, idx, gm;
    Tensor spill_list, spill_count;  // spill tiles (device list, device count)
    i64 tiles = 0;
    mutable int spills_host = -1;
    int host_spills() const;  // the spill count on the host (syncs once; only the opt-in one-kernel pre-activation asks)
  };
  std::map<std::pair<int, int>, HaloTable> halo;
  const HaloTable& halo_table(int B, int UM);
  // The brick hash, kept when built with keep_hash (for coordinate lookups by other consumers): slot table,
  // brick records, slot mask and the grid bounds.
  Tensor htable, hbricks;
  uint32_t hmask = 0;  // the table's slot mask, or (when hmaskd is set) its allocated capacity - 1
  Tensor hmaskd;       // device u32 mask of large tables (sized on the device from the brick count)
  int W = 0, H = 0, D = 0;
};
// coords int32 [N,4] (b,x,y,z); keep_hash keeps the brick hash in the cache (~32-128 B + 256 B per voxel) so that
// lookup() can answer arbitrary coordinate queries.
// The four-argument form is the reference's exact signature (src/spconv.h:12), so an object compiled against the
// reference header links against this library unchanged.
SpConvCache build_neighbors(const Tensor& coords, int W, int H, int D);
SpConvCache build_neighbors(const Tensor& coords, int W, int H, int D, bool keep_hash);

// Row of each query coordinate (b,x,y,z) in the cache's voxel set, -1 when absent or outside [0,W)x[0,H)x[0,D)
// (b < 0 included). The cache must have been built with keep_hash. Reference: the voxel hash probes of
// mesh.cu:14-19 (vhash_find) and spconv.cu:22-36, answered by the brick hash.
void lookup(const SpConvCache& c, const Tensor& query, Tensor& rows);

// Trilinear sample map of points grid f32 [L,3] (continuous voxel coordinates; voxel i's centre at i + 0.5) in batch
// `batch` of a keep_hash cache: the 8 voxels around p - 0.5, corner v = dx*4 + dy*2 + dz, nb u32 [L,8] their rows
// (EMPTY when absent or off-grid) and wt f32 [L,8] the trilinear weights (0 for EMPTY corners; with `normalize`
// divided by the sum of the present ones). Reference: the bake's FlexGEMM neighbour map + weight builder on its
// own voxel hash (src/glb.cu:547-550).
void grid_sample_map(const SpConvCache& c, const Tensor& grid, int batch, bool normalize, Tensor& nb, Tensor& wt);
// y[i] = sum_v x[nb[i,v]] * wt[i,v] in v order by fused multiply-adds (EMPTY reads 0); x f32 [M,C], y f32 [L,C]
// (reference k_wsum, src/glb.cu:456-465,551-552).
void grid_sample_sum(const Tensor& x, const Tensor& nb, const Tensor& wt, Tensor& y);

// FlexiDualGrid quads from the kernel map, no hash probes (reference k_fdg_quads, src/mesh.cu:36-45): for voxel i
// and axis a (e = 3i + a), if h[i,3+a] > 0 and the 4 voxels at the axis' edge offsets (all inside the 3x3x3
// neighbourhood) exist, ok[e] = 1 and quad[e] = their rows, else ok[e] = 0 (quad[e] left untouched). h f32 [N,7],
// quad int32 [3N,4], ok int32 [3N]. Equal to the reference when the cache was built with W = H = D = R over one
// batch (the reference's mesh hash key ignores the batch).
void fdg_quads(const SpConvCache& c, const Tensor& h, Tensor& quad, Tensor& ok);

// Tile choice. The reference replays FlexGEMM's autotune table (src/spconv.cu:177-221); here the tile is fixed
// per channel width (B1 = rows per tile and per schedule block, BK = channels per K stage, S = 1).
struct SpConvCfg {
  int B1, BK, S;
};
SpConvCfg spconv_cfg(int N, int Ci, int Co);
// The reference's tile choice for (N, Ci, Co) replayed from a FlexGEMM autotune cache file, section `device`
// (src/spconv.cu:176-221); B1 = 128, BK = 64, S = 1 where the file has no entry, or an error when `strict` is set or
// the environment has T2_STRICT=1 (src/spconv.cu:219).
SpConvCfg spconv_cfg_autotune(const std::string& path, const std::string& device, i64 N, int Ci, int Co,
                              bool strict = false);

// Conv-kernel timing: while on, each conv call brackets its conv kernels (not the weight repack or first-call
// schedules) with HIP events on the library stream; kernel_times() waits for them and returns each call's kernel ms
// in call order. kernel_timing(true) clears the list. No counterpart in the reference (its apps time whole calls).
void kernel_timing(bool on);
std::vector<float> kernel_times();

// y = subm_conv3d(x, w, b): x fp16/bf16 [N,Ci], w same dtype [Co,27,Ci], b fp16/bf16/fp32 [Co] or null.
// Returns [N,Co] in x's dtype; fp32 accumulation, bias added to the fp32 sum before the single rounding.
Tensor subm_conv(const Tensor& x, const Tensor& w, const Tensor* b, SpConvCache& c);

enum SpAct : int { ACT_NONE = 0, ACT_SILU = 1 };
// Flag or'ed into a conv's act: fp16 rounding-compatible epilogue. Instead of one rounding of act(acc + b) + r, the
// reference's sequence of fp16 roundings (src/spconv.cu:141-143, then act_ / add_, src/ops.cu:79-82,105-113):
// y = f16(f16(acc) + b); y = f16(y / (1 + exp(-y))) for SiLU; y = f16(y + r). Needs fp16 x, w, out and an fp16 (or
// no) bias and residual.
constexpr int EPI_F16_COMPAT = 256;
// Fused epilogue: out[i] = act(sum_v W_v x[nbr[i,v]] + b) [+ residual[i]], rounded once to out's dtype.
// residual may be null; out must be a defined [N,Co] tensor of dtype F32, F16 or BF16.
void subm_conv_fused(const Tensor& x, const Tensor& w, const Tensor* b, const Tensor* residual, int act,
                     SpConvCache& c, Tensor& out);

// The reference's fp16 conv under a replayed FlexGEMM tile choice (spconv_cfg_autotune), rounding included: S == 1
// is subm_conv_fused with EPI_F16_COMPAT; S > 1 writes fp32 partials per split (the split's share of each B1
// block's K chunks, fp32 bias in split 0) and sums them with four interleaved accumulators before the one fp16
// rounding (src/spconv.cu:98-99,144-157), then act / residual as the reference's separate fp16 passes. fp16 only.
void subm_conv_replay(const Tensor& x, const Tensor& w, const Tensor* b, const Tensor* residual, int act,
                      const SpConvCfg& cfg, SpConvCache& c, Tensor& out);

// Conv of gathered rows without materializing them: out = subm_conv_fused(x_src[row_map >> shift], ...).
// x_src [M,Ci]; row_map int32 [N] (N = the cache's rows), e.g. the c2s parent map (src, shift 3), so a decoder's
// upsample block (reference src/sdec.cu:34-43 k_gather_rows then the conv at :70-87) reads the parent rows
// directly. Entries outside [0, M) read as zero rows.
void subm_conv_gathered(const Tensor& x_src, const Tensor& row_map, int shift, const Tensor& w, const Tensor* b,
                        const Tensor* residual, int act, SpConvCache& c, Tensor& out);

// Pre-activation of an upsample block's convs in one pass (reference src/sdec.cu:72-73, 78-83): out[i] =
// act(LayerNorm(x_src[row_map[i] >> shift]) * gamma + beta) with fp32 statistics and one rounding; x_src bf16/fp16
// [M,C], out [N,C] of the same dtype, gamma/beta f32 [C] or null, act ACT_NONE / ACT_SILU. Map entries outside
// [0,M) read zero rows; a null row_map is the identity (N = M).
void gather_ln_act(const Tensor& x_src, const Tensor* row_map, int shift, const Tensor* gamma, const Tensor* beta,
                   float eps, int act, Tensor& out);

// ConvNeXt tail of the decoder in one pass (reference SDecoder::convnext after its conv, src/sdec.cu:60-66):
// y = x + W2 silu(W1 (LayerNorm(h) * gamma + beta) + b1) + b2 per row, LayerNorm eps as given, fp32 accumulation,
// hidden activations rounded to h's dtype between the two products. h, x, y [N,C] and w1 [4C,C], w2 [C,4C] of one
// dtype (fp16/bf16); gamma, beta, b2 [C] and b1 [4C] of any float dtype or null; C = 64, 128 or 256 in one pass,
// C = 512 or 1024 (the coarse levels) as LayerNorm + two GEMMs with fused epilogues. y may alias h or x.
void convnext_mlp(const Tensor& h, const Tensor& x, const Tensor* gamma, const Tensor* beta, float eps, const Tensor& w1,
                  const Tensor* b1, const Tensor& w2, const Tensor* b2, Tensor& y);

// Conv plus the upsample block's skip connection in one pass: out = act(conv(x) + b) + skip, skip[i, c] =
// x_skip[src[i] >> 3, (src[i] & 7) * Cin/8 + c / rep], rep = Co / (Cin/8) a power of two, one rounding (reference:
// subm_conv then k_add_skip, src/sdec.cu:38-43, 82-84). Fused into the 64 -> 64 halo kernel; other shapes run the
// conv and then add_skip. out and x_skip share a 16-bit dtype.
void subm_conv_skip(const Tensor& x, const Tensor& w, const Tensor* b, int act, const Tensor& x_skip,
                    const Tensor& src, SpConvCache& c, Tensor& out);

// Conv of pre-activated rows (the upsample block's norm2 + SiLU + conv2 + skip, reference src/sdec.cu:78-84, or
// any LayerNorm -> act -> conv): x = act_pre(LayerNorm(x_src[row_map >> shift]) * gamma + beta) (row_map null: the
// rows of x_src, which then has the cache's rows), out = act(conv(x, w) + b) [+ the skip of subm_conv_skip when
// x_skip / skip_src are given]: gather_ln_act and then the conv; with SPCONV_PRELN_FUSED set, 64-output-channel
// convs served by the halo kernel without spill tiles run it as one kernel instead (the pre-activation applied to
// each tile's halo rows in LDS; slower, see conv.hip). Same bits either way. x_src, w, x_skip, out: one 16-bit
// dtype; gamma / beta f32 [Ci] or null.
void subm_conv_preln(const Tensor& x_src, const Tensor* row_map, int shift, const Tensor* gamma, const Tensor* beta,
                     float eps, int pre_act, const Tensor& w, const Tensor* b, int act, const Tensor* x_skip,
                     const Tensor* skip_src, SpConvCache& c, Tensor& out);

// Skip connection of the upsample block, in place (reference k_add_skip, src/sdec.cu:38-43):
// h[i, c] += x[src[i] >> 3, (src[i] & 7) * Cin/8 + c / rep], rep = Co / (Cin/8), fp32 sum rounded once (bit-identical
// to the reference). h [m,Co] and x [n,Cin] of one dtype (fp16/bf16); entries of src outside x leave the row.
void add_skip(Tensor& h, const Tensor& x, const Tensor& src);

// out[i] = row_map[tbl[i]] >> shift for every entry of a neighbour table, EMPTY where tbl[i] is EMPTY or the
// mapped row is not below m (the row-map form of a tile-order table, for the gathered conv).
void map_table_rows(const Tensor& tbl, const Tensor& row_map, int shift, i64 m, Tensor& out);

// Child subdivision of a sparse level (reference src/sdec.cu:20-57): children of each parent whose fp16 logit is
// > 0, in (parent, slot) order, coords (b, 2x+(s&1), 2y+(s>>1&1), 2z+(s>>2&1)), src = parent*8+s.
struct Subdivision {
  Tensor coords, src;  // int32 [M,4], int32 [M]
};
Subdivision subdivide(const Tensor& coords, const Tensor& logits_f16);
// Subdivision and the children's kernel map with no host sync in between (the reference waits for the child count
// at src/sdec.cu:52 before it can size the map): every launch is sized for the 8n-child capacity and its kernels stop
// at the count on the device; the count is copied back while the map build runs and read once all of it is queued.
// coords_out / src_out: optional caller buffers of >= 8n rows (else allocated). The cache equals
// build_neighbors(coords, W, H, D) on the children.
struct UpsampleLevel {
  Tensor coords, src;  // int32 [M,4], int32 [M] (views of the capacity buffers)
  SpConvCache cache;
};
UpsampleLevel subdivide_build(const Tensor& coords, const Tensor& logits_f16, int W, int H, int D,
                              int32_t* coords_out = nullptr, int32_t* src_out = nullptr);
// The same children written into caller buffers of >= 8n rows, the count into device memory (*m_dev, int64), with no
// allocation and no host sync: its scratch is a static device array whose device address is looked up on a
// device's first call, so n <= the maximum below and concurrent calls on one GPU race.
i64 subdivide_noalloc_max_parents();
void subdivide_noalloc(const int32_t* coords, const uint16_t* logits_f16, i64 n, int32_t* child_coords, int32_t* src,
                       i64* m_dev);

#pragma GCC visibility pop
