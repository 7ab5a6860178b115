// PyTorch operator registration of the prism_bsa C-ABI: TORCH_LIBRARY(prism).
//
// Every operator is a thin wrapper of one extern "C" entry point of
// include/prism_bsa.h: it checks devices and dtypes, allocates its outputs
// through the caching allocator (at::empty on the inputs' device), and
// launches on the current HIP stream of that device.  Errors of the C-ABI
// come back as ValueError (invalid argument) or RuntimeError (launch error),
// as the reference raises them from its Python host layer.  Operators that
// produce an optional output return an empty tensor when it is not asked for.
//
// The schemas follow the host-side calls of the reference's block-sparse
// path (hymm/models/modules/block_sparse_attention/): zone statistics and
// shapes (dynamic_block_shape.py:68-355), the A2V norms (wan_video_dit.py:
// 742-752), geometry (dynamic_block_attention.py:107-170), gathers + pooling
// (:250-268, bsa_interface.py:164-201), scores + selection (bsa_interface.py:
// 203-304), the list transpose (:147-161) and the attention kernels
// (:328-523); each entry point's header comment cites its function.
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include "../../include/prism_bsa.h"

namespace {

using at::Tensor;
using OptT = c10::optional<Tensor>;

// the C-ABI's messages start with the entry point's name
void check_rc(int rc) {
  if (rc == 1) TORCH_CHECK_VALUE(false, prism_last_error());
  TORCH_CHECK(rc == 0, prism_last_error());
}
#define PRISM_TORCH_CALL(fn, ...) check_rc(fn(__VA_ARGS__))

hipStream_t stream_of(const Tensor& t) { return c10::hip::getCurrentHIPStream(t.device().index()).stream(); }

void on_gpu(const Tensor& t, const char* name) {
  TORCH_CHECK_VALUE(t.defined() && t.is_cuda(), "prism: ", name, " must be a GPU tensor (no CPU path)");
}
void on_gpu(const OptT& t, const char* name) {
  if (t && t->defined()) on_gpu(*t, name);
}

const void* p(const OptT& t) { return t && t->defined() ? t->data_ptr() : nullptr; }
OptT cont(const OptT& t) { return t && t->defined() ? OptT(t->contiguous()) : OptT(); }

int dtype_code(const Tensor& t) {
  if (t.scalar_type() == at::kFloat) return PRISM_F32;
  if (t.scalar_type() == at::kBFloat16) return PRISM_BF16;
  TORCH_CHECK_TYPE(false, "prism: unsupported dtype ", t.scalar_type(), " (float32 or bfloat16)");
  return -1;
}
at::ScalarType dtype_of_code(int64_t c) {
  TORCH_CHECK_VALUE(c == PRISM_F32 || c == PRISM_BF16, "prism: dtype code ", c, " unknown");
  return c == PRISM_F32 ? at::kFloat : at::kBFloat16;
}
void check_dtype(const Tensor& t, at::ScalarType s, const char* name) {
  TORCH_CHECK_TYPE(t.scalar_type() == s, "prism: ", name, " must be ", s, ", got ", t.scalar_type());
}
void check_dtype(const OptT& t, at::ScalarType s, const char* name) {
  if (t && t->defined()) check_dtype(*t, s, name);
}
at::TensorOptions opts(const Tensor& like, at::ScalarType s) { return like.options().dtype(s); }
Tensor none_like(const Tensor& like) { return at::empty({0}, opts(like, at::kFloat)); }

int64_t zones(c10::IntArrayRef g) {
  TORCH_CHECK_VALUE(g.size() == 3, "prism: a grid has three extents");
  return (g[0] / 8) * (g[1] / 8) * (g[2] / 8);
}

// ------------------------------------------------------------------ statistics
std::tuple<Tensor, Tensor> zone_stats(const Tensor& v_, const OptT& valid_, c10::IntArrayRef grid,
                                      c10::IntArrayRef box) {
  on_gpu(v_, "v");
  on_gpu(valid_, "valid");
  check_dtype(valid_, at::kByte, "valid");
  const c10::DeviceGuard guard(v_.device());
  const Tensor v = v_.contiguous();
  const OptT valid = cont(valid_);
  TORCH_CHECK_VALUE(v.dim() == 4, "zone_stats: v must be [B,H,S,D]");
  const int64_t Nz = zones(grid), D = v.size(3);
  Tensor packed = at::empty({Nz, 25 * D}, opts(v, at::kFloat));
  Tensor av = at::empty({Nz, 24}, opts(v, at::kByte));
  PRISM_TORCH_CALL(prism_zone_stats, v.data_ptr(), dtype_code(v), (int)v.size(1), v.size(2), (int)D,
                   (const uint8_t*)p(valid), (int)grid[0], (int)grid[1], (int)grid[2], (int)box[0], (int)box[1],
                   (int)box[2], packed.data_ptr<float>(), av.data_ptr<uint8_t>(), stream_of(v));
  return {packed, av};
}

std::tuple<Tensor, Tensor> audio_zone_stats(const Tensor& norms_, const OptT& valid_, c10::IntArrayRef grid,
                                            c10::IntArrayRef box) {
  on_gpu(norms_, "norms");
  on_gpu(valid_, "valid");
  check_dtype(valid_, at::kByte, "valid");
  const c10::DeviceGuard guard(norms_.device());
  const Tensor n = norms_.contiguous();
  const OptT valid = cont(valid_);
  const int64_t Nz = zones(grid);
  Tensor abar = at::empty({Nz}, opts(n, at::kFloat));
  Tensor vhat = at::empty({Nz, 3}, opts(n, at::kFloat));
  PRISM_TORCH_CALL(prism_audio_zone_stats, n.data_ptr(), dtype_code(n), (const uint8_t*)p(valid), (int)grid[0],
                   (int)grid[1], (int)grid[2], (int)box[0], (int)box[1], (int)box[2], abar.data_ptr<float>(),
                   vhat.data_ptr<float>(), stream_of(n));
  return {abar, vhat};
}

std::tuple<Tensor, Tensor> zone_gradient(const Tensor& packed_, const Tensor& av_, int64_t D) {
  on_gpu(packed_, "packed");
  on_gpu(av_, "axis_valid");
  check_dtype(packed_, at::kFloat, "packed");
  check_dtype(av_, at::kByte, "axis_valid");
  const c10::DeviceGuard guard(packed_.device());
  const Tensor packed = packed_.contiguous(), av = av_.contiguous();
  const int64_t Nz = packed.size(0);
  Tensor rho_raw = at::empty({Nz}, opts(packed, at::kFloat));
  Tensor aniso = at::empty({Nz, 3}, opts(packed, at::kFloat));
  PRISM_TORCH_CALL(prism_zone_gradient, packed.data_ptr<float>(), av.data_ptr<uint8_t>(), (int)Nz, (int)D,
                   rho_raw.data_ptr<float>(), aniso.data_ptr<float>(), stream_of(packed));
  return {rho_raw, aniso};
}

std::tuple<Tensor, Tensor, Tensor> zone_shapes(const Tensor& rho_raw_, const Tensor& aniso_, const OptT& abar_,
                                               const OptT& vhat_, int64_t method, double lambda_a, double tau_128,
                                               double lambda_128) {
  on_gpu(rho_raw_, "rho_raw");
  on_gpu(aniso_, "aniso");
  on_gpu(abar_, "abar");
  on_gpu(vhat_, "vhat");
  const c10::DeviceGuard guard(rho_raw_.device());
  const Tensor rho_raw = rho_raw_.contiguous(), aniso = aniso_.contiguous();
  const OptT abar = cont(abar_), vhat = cont(vhat_);
  const int64_t Nz = rho_raw.size(0);
  Tensor g = at::empty({Nz, 3}, opts(rho_raw, at::kFloat));
  Tensor rho = at::empty({Nz}, opts(rho_raw, at::kFloat));
  Tensor sid = at::empty({Nz}, opts(rho_raw, at::kLong));
  PRISM_TORCH_CALL(prism_zone_shapes, rho_raw.data_ptr<float>(), aniso.data_ptr<float>(), (const float*)p(abar),
                   (const float*)p(vhat), (int)Nz, (int)method, (float)lambda_a, (float)tau_128, (float)lambda_128,
                   g.data_ptr<float>(), rho.data_ptr<float>(), sid.data_ptr<int64_t>(), stream_of(rho_raw));
  return {g, rho, sid};
}

Tensor assign_shapes(const Tensor& g_, const Tensor& rho_, int64_t method, double tau_128, double lambda_128) {
  on_gpu(g_, "g");
  on_gpu(rho_, "rho");
  check_dtype(g_, at::kFloat, "g");
  check_dtype(rho_, at::kFloat, "rho");
  const c10::DeviceGuard guard(g_.device());
  const Tensor g = g_.contiguous(), rho = rho_.contiguous();
  const int64_t Nz = rho.size(0);
  Tensor sid = at::empty({Nz}, opts(g, at::kLong));
  PRISM_TORCH_CALL(prism_assign_shapes, g.data_ptr<float>(), rho.data_ptr<float>(), (int)Nz, (int)method,
                   (float)tau_128, (float)lambda_128, sid.data_ptr<int64_t>(), stream_of(g));
  return sid;
}

Tensor a2v_norms(const Tensor& res_) {
  on_gpu(res_, "residual");
  const c10::DeviceGuard guard(res_.device());
  const Tensor r = res_.contiguous();
  TORCH_CHECK_VALUE(r.dim() == 2, "a2v_norms: residual must be [S, C]");
  Tensor out = at::empty({r.size(0)}, r.options());
  PRISM_TORCH_CALL(prism_a2v_norms, r.data_ptr(), dtype_code(r), r.size(0), (int)r.size(1), out.data_ptr(),
                   dtype_code(out), stream_of(r));
  return out;
}

std::tuple<Tensor, Tensor> linear_rownorm(const Tensor& x_, const Tensor& w_, const OptT& bias_, int64_t norms_dtype) {
  on_gpu(x_, "x");
  on_gpu(w_, "weight");
  on_gpu(bias_, "bias");
  check_dtype(x_, at::kBFloat16, "x");
  check_dtype(w_, at::kBFloat16, "weight");
  check_dtype(bias_, at::kBFloat16, "bias");
  const c10::DeviceGuard guard(x_.device());
  const Tensor x = x_.contiguous(), w = w_.contiguous();
  const OptT bias = cont(bias_);
  TORCH_CHECK_VALUE(x.dim() == 2 && w.dim() == 2 && w.size(1) == x.size(1),
                    "linear_rownorm: x must be [M, K] and weight [N, K]");
  if (bias) TORCH_CHECK_VALUE(bias->numel() == w.size(0), "linear_rownorm: bias must have N entries");
  const int64_t M = x.size(0), N = w.size(0), K = x.size(1);
  Tensor y = at::empty({M, N}, x.options());
  Tensor norms = at::empty({M}, opts(x, dtype_of_code(norms_dtype)));
  Tensor partial = at::empty({M * std::max<int64_t>(N / 256, 1)}, opts(x, at::kFloat));
  PRISM_TORCH_CALL(prism_linear_rownorm, x.data_ptr(), w.data_ptr(), p(bias), M, (int)N, (int)K, y.data_ptr(),
                   norms.data_ptr(), (int)norms_dtype, partial.data_ptr<float>(), stream_of(x));
  return {y, norms};
}

// ------------------------------------------------------------------ geometry
std::tuple<Tensor, Tensor, Tensor> zone_layout(const Tensor& sid_) {
  on_gpu(sid_, "shape_ids");
  check_dtype(sid_, at::kLong, "shape_ids");
  const c10::DeviceGuard guard(sid_.device());
  const Tensor sid = sid_.contiguous();
  const int64_t Nz = sid.numel();
  Tensor boff = at::empty({Nz + 1}, opts(sid, at::kInt));
  Tensor bot = at::empty({Nz * 8}, opts(sid, at::kInt));
  Tensor bft = at::empty({Nz * 8 + 1}, opts(sid, at::kInt));
  PRISM_TORCH_CALL(prism_zone_layout, sid.data_ptr<int64_t>(), (int)Nz, boff.data_ptr<int32_t>(),
                   bot.data_ptr<int32_t>(), bft.data_ptr<int32_t>(), stream_of(sid));
  return {boff, bot, bft};
}

std::tuple<Tensor, Tensor> rearrange_index(const Tensor& sid_, c10::IntArrayRef grid) {
  on_gpu(sid_, "shape_ids");
  check_dtype(sid_, at::kLong, "shape_ids");
  const c10::DeviceGuard guard(sid_.device());
  const Tensor sid = sid_.contiguous();
  const int64_t S = grid[0] * grid[1] * grid[2];
  Tensor src = at::empty({S}, opts(sid, at::kLong));
  Tensor inv = at::empty({S}, opts(sid, at::kLong));
  PRISM_TORCH_CALL(prism_rearrange_index, sid.data_ptr<int64_t>(), (int)grid[0], (int)grid[1], (int)grid[2],
                   src.data_ptr<int64_t>(), inv.data_ptr<int64_t>(), stream_of(sid));
  return {src, inv};
}

// outputs of the gathers: rows, block_mean, block_count, tile_count, valid_re, rowdot
using Gathered = std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor>;

Gathered gathered(const Tensor& x, int64_t B, int64_t H, int64_t S_out, int64_t D, int64_t N_b, int64_t Nt,
                  bool rows, bool pool, bool counts, bool rowdot) {
  return {rows ? at::empty({B, H, S_out, D}, opts(x, at::kBFloat16)) : none_like(x),
          pool ? at::empty({B, H, N_b, D}, opts(x, at::kFloat)) : none_like(x),
          counts ? at::empty({N_b}, opts(x, at::kInt)) : none_like(x),
          counts ? at::empty({Nt}, opts(x, at::kInt)) : none_like(x),
          counts ? at::empty({S_out}, opts(x, at::kByte)) : none_like(x),
          rowdot ? at::empty({B, H, S_out}, opts(x, at::kFloat)) : none_like(x)};
}
void* maybe(const Tensor& t) { return t.numel() ? t.data_ptr() : nullptr; }

Gathered gather_pool(const Tensor& x_, const OptT& valid_, const Tensor& sid_, const Tensor& boff_,
                     c10::IntArrayRef grid, c10::IntArrayRef box, int64_t N_b, bool rows, bool pool, bool counts,
                     const OptT& dot_) {
  on_gpu(x_, "x");
  on_gpu(valid_, "valid");
  on_gpu(sid_, "shape_ids");
  on_gpu(boff_, "block_offset");
  on_gpu(dot_, "dot_with");
  check_dtype(valid_, at::kByte, "valid");
  check_dtype(sid_, at::kLong, "shape_ids");
  check_dtype(boff_, at::kInt, "block_offset");
  check_dtype(dot_, at::kBFloat16, "dot_with");
  const c10::DeviceGuard guard(x_.device());
  const Tensor x = x_.contiguous(), sid = sid_.contiguous(), boff = boff_.contiguous();
  const OptT valid = cont(valid_), dot = cont(dot_);
  TORCH_CHECK_VALUE(x.dim() == 4, "gather_pool: x must be [B,H,S,D]");
  const int64_t B = x.size(0), H = x.size(1), D = x.size(3), S = grid[0] * grid[1] * grid[2];
  Gathered o = gathered(x, B, H, S, D, N_b, S / 64, rows, pool, counts, dot.has_value());
  if (dot) TORCH_CHECK_VALUE(dot->sizes() == at::IntArrayRef({B, H, S, D}), "gather_pool: dot_with must be [B,H,S,D]");
  PRISM_TORCH_CALL(prism_gather_pool, x.data_ptr(), dtype_code(x), (int)B, (int)H, x.size(2), (int)D,
                   (const uint8_t*)p(valid), sid.data_ptr<int64_t>(), boff.data_ptr<int32_t>(), (int)grid[0],
                   (int)grid[1], (int)grid[2], (int)box[0], (int)box[1], (int)box[2], N_b, maybe(std::get<0>(o)),
                   (float*)maybe(std::get<1>(o)), (int32_t*)maybe(std::get<2>(o)), (int32_t*)maybe(std::get<3>(o)),
                   (uint8_t*)maybe(std::get<4>(o)), p(dot), (float*)maybe(std::get<5>(o)), stream_of(x));
  return o;
}

Tensor scatter_rows(const Tensor& rows_, const Tensor& sid_, c10::IntArrayRef grid, c10::IntArrayRef box,
                    int64_t out_dtype) {
  on_gpu(rows_, "rows");
  on_gpu(sid_, "shape_ids");
  check_dtype(rows_, at::kBFloat16, "rows");
  check_dtype(sid_, at::kLong, "shape_ids");
  const c10::DeviceGuard guard(rows_.device());
  const Tensor rows = rows_.contiguous(), sid = sid_.contiguous();
  TORCH_CHECK_VALUE(rows.dim() == 4, "scatter_rows: rows must be [B,H,S,D]");
  const int64_t S_in = box[0] * box[1] * box[2];
  Tensor out = at::empty({rows.size(0), rows.size(1), S_in, rows.size(3)}, opts(rows, dtype_of_code(out_dtype)));
  PRISM_TORCH_CALL(prism_scatter_rows, rows.data_ptr(), (int)rows.size(0), (int)rows.size(1), S_in, (int)rows.size(3),
                   sid.data_ptr<int64_t>(), (int)grid[0], (int)grid[1], (int)grid[2], (int)box[0], (int)box[1],
                   (int)box[2], out.data_ptr(), (int)out_dtype, stream_of(rows));
  return out;
}

Gathered chunk_gather_pool(const Tensor& x_, const OptT& valid_, c10::IntArrayRef grid, c10::IntArrayRef pgrid,
                           c10::IntArrayRef chunk, int64_t S_out, bool rows, bool pool, bool counts,
                           const OptT& dot_) {
  on_gpu(x_, "x");
  on_gpu(valid_, "valid");
  on_gpu(dot_, "dot_with");
  check_dtype(valid_, at::kByte, "valid");
  check_dtype(dot_, at::kBFloat16, "dot_with");
  const c10::DeviceGuard guard(x_.device());
  const Tensor x = x_.contiguous();
  const OptT valid = cont(valid_), dot = cont(dot_);
  TORCH_CHECK_VALUE(x.dim() == 4, "chunk_gather_pool: x must be [B,H,S,D]");
  TORCH_CHECK_VALUE(grid.size() == 3 && pgrid.size() == 3 && chunk.size() == 3, "chunk_gather_pool: 3-D extents");
  const int64_t B = x.size(0), H = x.size(1), D = x.size(3);
  const int64_t csz = chunk[0] * chunk[1] * chunk[2];
  TORCH_CHECK_VALUE(csz > 0, "chunk_gather_pool: empty chunk");
  const int64_t N_b = pgrid[0] * pgrid[1] * pgrid[2] / csz;
  Gathered o = gathered(x, B, H, S_out, D, N_b, S_out / 64, rows, pool, counts, dot.has_value());
  if (dot)
    TORCH_CHECK_VALUE(dot->sizes() == at::IntArrayRef({B, H, S_out, D}), "chunk_gather_pool: dot_with must be [B,H,S_out,D]");
  PRISM_TORCH_CALL(prism_chunk_gather_pool, x.data_ptr(), dtype_code(x), (int)B, (int)H, (int)D,
                   (const uint8_t*)p(valid), (int)grid[0], (int)grid[1], (int)grid[2], (int)pgrid[0], (int)pgrid[1],
                   (int)pgrid[2], (int)chunk[0], (int)chunk[1], (int)chunk[2], S_out, maybe(std::get<0>(o)),
                   (float*)maybe(std::get<1>(o)), (int32_t*)maybe(std::get<2>(o)), (int32_t*)maybe(std::get<3>(o)),
                   (uint8_t*)maybe(std::get<4>(o)), p(dot), (float*)maybe(std::get<5>(o)), stream_of(x));
  return o;
}

Tensor chunk_scatter_rows(const Tensor& rows_, c10::IntArrayRef grid, c10::IntArrayRef pgrid, c10::IntArrayRef chunk,
                          int64_t out_dtype) {
  on_gpu(rows_, "rows");
  check_dtype(rows_, at::kBFloat16, "rows");
  const c10::DeviceGuard guard(rows_.device());
  const Tensor rows = rows_.contiguous();
  TORCH_CHECK_VALUE(rows.dim() == 4, "chunk_scatter_rows: rows must be [B,H,S_out,D]");
  const int64_t S_in = grid[0] * grid[1] * grid[2];
  Tensor out = at::empty({rows.size(0), rows.size(1), S_in, rows.size(3)}, opts(rows, dtype_of_code(out_dtype)));
  PRISM_TORCH_CALL(prism_chunk_scatter_rows, rows.data_ptr(), (int)rows.size(0), (int)rows.size(1), (int)rows.size(3),
                   (int)grid[0], (int)grid[1], (int)grid[2], (int)pgrid[0], (int)pgrid[1], (int)pgrid[2],
                   (int)chunk[0], (int)chunk[1], (int)chunk[2], rows.size(2), out.data_ptr(), (int)out_dtype,
                   stream_of(rows));
  return out;
}

// ------------------------------------------------------------------ selection
Tensor block_scores(const Tensor& qc_, const Tensor& kc_, const OptT& bc_) {
  on_gpu(qc_, "qc");
  on_gpu(kc_, "kc");
  on_gpu(bc_, "block_count");
  check_dtype(qc_, at::kFloat, "qc");
  check_dtype(kc_, at::kFloat, "kc");
  check_dtype(bc_, at::kInt, "block_count");
  const c10::DeviceGuard guard(qc_.device());
  const Tensor qc = qc_.contiguous(), kc = kc_.contiguous();
  const OptT bc = cont(bc_);
  TORCH_CHECK_VALUE(qc.dim() >= 2 && kc.dim() >= 2, "block_scores: means must be [..., N, D]");
  const int64_t Nq = qc.size(-2), D = qc.size(-1), Nk = kc.size(-2);
  const int64_t BH = Nq * D ? qc.numel() / (Nq * D) : 0;
  TORCH_CHECK_VALUE(kc.size(-1) == D && kc.numel() == BH * Nk * D, "block_scores: q and k means must share batch dims and D");
  std::vector<int64_t> shape(qc.sizes().begin(), qc.sizes().end() - 1);
  shape.push_back(Nk);
  Tensor out = at::empty(shape, opts(qc, at::kFloat));
  PRISM_TORCH_CALL(prism_block_scores, qc.data_ptr<float>(), kc.data_ptr<float>(), (const int32_t*)p(bc), (int)BH, Nq,
                   Nk, (int)D, out.data_ptr<float>(), stream_of(qc));
  return out;
}

std::tuple<Tensor, Tensor, Tensor, Tensor> select_tiles(const Tensor& scores_, int64_t mode, int64_t k_lo, int64_t ub,
                                                        double scale, int64_t thr, const Tensor& bft_,
                                                        const OptT& tcount_, int64_t tcap, int64_t bcap,
                                                        bool want_blocks) {
  on_gpu(scores_, "scores");
  on_gpu(bft_, "block_first_tile");
  on_gpu(tcount_, "tile_count");
  check_dtype(scores_, at::kFloat, "scores");
  check_dtype(bft_, at::kInt, "block_first_tile");
  check_dtype(tcount_, at::kInt, "tile_count");
  TORCH_CHECK_VALUE(thr >= 0, "select_tiles: threshold must be >= 0");
  const c10::DeviceGuard guard(scores_.device());
  const Tensor scores = scores_.contiguous(), bft = bft_.contiguous();
  const OptT tcount = cont(tcount_);
  const int64_t N = scores.size(-1), rows = N ? scores.numel() / N : 0;
  Tensor tiles = at::empty({rows, tcap}, opts(scores, at::kInt));
  Tensor ntiles = at::empty({rows}, opts(scores, at::kInt));
  Tensor sel = want_blocks ? at::full({rows, bcap}, N, opts(scores, at::kInt)) : none_like(scores);
  Tensor nsel = want_blocks ? at::empty({rows}, opts(scores, at::kInt)) : none_like(scores);
  PRISM_TORCH_CALL(prism_select_tiles, scores.data_ptr<float>(), rows, N, (int)mode, k_lo, ub, (float)scale,
                   (uint64_t)thr, bft.data_ptr<int32_t>(), (const int32_t*)p(tcount), tcap, tiles.data_ptr<int32_t>(),
                   ntiles.data_ptr<int32_t>(), (int32_t*)maybe(sel), bcap, (int32_t*)maybe(nsel), stream_of(scores));
  return {tiles, ntiles, sel, nsel};
}

std::tuple<Tensor, Tensor> tile_rows(const Tensor& ntiles_, const Tensor& bot_, const OptT& qtc_, int64_t BH,
                                     int64_t Nt, int64_t N_b, int64_t tcap) {
  on_gpu(ntiles_, "ntiles");
  on_gpu(bot_, "block_id_of_tile");
  on_gpu(qtc_, "q_tile_count");
  check_dtype(ntiles_, at::kInt, "ntiles");
  check_dtype(bot_, at::kInt, "block_id_of_tile");
  check_dtype(qtc_, at::kInt, "q_tile_count");
  const c10::DeviceGuard guard(ntiles_.device());
  const Tensor ntiles = ntiles_.contiguous(), bot = bot_.contiguous();
  const OptT qtc = cont(qtc_);
  Tensor qstart = at::empty({BH * Nt}, opts(ntiles, at::kLong));
  Tensor qlen = at::empty({BH * Nt}, opts(ntiles, at::kInt));
  PRISM_TORCH_CALL(prism_tile_rows, ntiles.data_ptr<int32_t>(), bot.data_ptr<int32_t>(), (const int32_t*)p(qtc),
                   (int)BH, Nt, N_b, tcap, qstart.data_ptr<int64_t>(), qlen.data_ptr<int32_t>(), stream_of(ntiles));
  return {qstart, qlen};
}

void check_lists(const Tensor& start, const Tensor& len, const Tensor& cols) {
  on_gpu(start, "start");
  on_gpu(len, "len");
  on_gpu(cols, "cols");
  check_dtype(start, at::kLong, "start");
  check_dtype(len, at::kInt, "len");
  check_dtype(cols, at::kInt, "cols");
}

std::tuple<Tensor, Tensor, Tensor> transpose_lists(const Tensor& qs_, const Tensor& ql_, const Tensor& qc_,
                                                   int64_t BH, int64_t Ntq, int64_t Ntk) {
  check_lists(qs_, ql_, qc_);
  const c10::DeviceGuard guard(qs_.device());
  const Tensor qs = qs_.contiguous(), ql = ql_.contiguous(), qc = qc_.contiguous();
  const int64_t words = (Ntq + 31) / 32;
  Tensor bitmap = at::empty({BH * Ntk * words}, opts(qs, at::kInt));
  Tensor kstart = at::empty({BH * Ntk}, opts(qs, at::kLong));
  Tensor klen = at::empty({BH * Ntk}, opts(qs, at::kInt));
  Tensor kcols = at::empty({BH * Ntk * Ntq}, opts(qs, at::kInt));
  PRISM_TORCH_CALL(prism_transpose_lists, qs.data_ptr<int64_t>(), ql.data_ptr<int32_t>(), qc.data_ptr<int32_t>(),
                   (int)BH, Ntq, Ntk, (uint32_t*)bitmap.data_ptr<int32_t>(), Ntq, kstart.data_ptr<int64_t>(),
                   klen.data_ptr<int32_t>(), kcols.data_ptr<int32_t>(), stream_of(qs));
  return {kstart, klen, kcols};
}

// ------------------------------------------------------------------ attention work lists
Tensor pair_tiles(const Tensor& s_, const Tensor& l_, const Tensor& c_, int64_t row_tiles, int64_t col_tiles) {
  check_lists(s_, l_, c_);
  const c10::DeviceGuard guard(s_.device());
  const Tensor s = s_.contiguous(), l = l_.contiguous(), c = c_.contiguous();
  Tensor out = at::empty({s.numel()}, opts(s, at::kInt));
  PRISM_TORCH_CALL(prism_pair_tiles, s.data_ptr<int64_t>(), l.data_ptr<int32_t>(), c.data_ptr<int32_t>(), s.numel(),
                   row_tiles, col_tiles, out.data_ptr<int32_t>(), stream_of(s));
  return out;
}

std::tuple<Tensor, Tensor, Tensor> pair_union(const Tensor& s_, const Tensor& l_, const Tensor& c_, int64_t row_tiles,
                                              int64_t col_tiles, const OptT& pairmap_, const OptT& masks_) {
  check_lists(s_, l_, c_);
  on_gpu(pairmap_, "pairmap");
  on_gpu(masks_, "tile_masks");
  check_dtype(pairmap_, at::kInt, "pairmap");
  check_dtype(masks_, at::kLong, "tile_masks");
  const c10::DeviceGuard guard(s_.device());
  const Tensor s = s_.contiguous(), l = l_.contiguous(), c = c_.contiguous();
  const OptT pairmap = cont(pairmap_), masks = cont(masks_);
  const int64_t rows = s.numel(), pairs = rows / 2;
  Tensor ustart = at::empty({pairs}, opts(s, at::kLong));
  Tensor ulen = at::empty({pairs}, opts(s, at::kInt));
  Tensor ucols = at::empty({std::max<int64_t>(pairs * col_tiles, 1)}, opts(s, at::kInt));
  PRISM_TORCH_CALL(prism_pair_union, s.data_ptr<int64_t>(), l.data_ptr<int32_t>(), c.data_ptr<int32_t>(), rows,
                   row_tiles, col_tiles, (const int32_t*)p(pairmap), (const uint64_t*)p(masks), col_tiles,
                   ustart.data_ptr<int64_t>(), ulen.data_ptr<int32_t>(), ucols.data_ptr<int32_t>(), stream_of(s));
  return {ustart, ulen, ucols};
}

// quad unions: rows of four tiles (pairmap[4 q + k]), entries
// tile << 5 | partial << 4 | member bits
std::tuple<Tensor, Tensor, Tensor> quad_union(const Tensor& s_, const Tensor& l_, const Tensor& c_, int64_t row_tiles,
                                              int64_t col_tiles, const OptT& pairmap_, const OptT& masks_) {
  check_lists(s_, l_, c_);
  on_gpu(pairmap_, "pairmap");
  on_gpu(masks_, "tile_masks");
  check_dtype(pairmap_, at::kInt, "pairmap");
  check_dtype(masks_, at::kLong, "tile_masks");
  const c10::DeviceGuard guard(s_.device());
  const Tensor s = s_.contiguous(), l = l_.contiguous(), c = c_.contiguous();
  const OptT pairmap = cont(pairmap_), masks = cont(masks_);
  const int64_t rows = s.numel(), quads = rows / 4;
  Tensor ustart = at::empty({quads}, opts(s, at::kLong));
  Tensor ulen = at::empty({quads}, opts(s, at::kInt));
  Tensor ucols = at::empty({std::max<int64_t>(quads * col_tiles, 1)}, opts(s, at::kInt));
  PRISM_TORCH_CALL(prism_quad_union, s.data_ptr<int64_t>(), l.data_ptr<int32_t>(), c.data_ptr<int32_t>(), rows,
                   row_tiles, col_tiles, (const int32_t*)p(pairmap), (const uint64_t*)p(masks), col_tiles,
                   ustart.data_ptr<int64_t>(), ulen.data_ptr<int32_t>(), ucols.data_ptr<int32_t>(), stream_of(s));
  return {ustart, ulen, ucols};
}

// CSR entry buffer of nnz entries, with at least one element: lists that
// hold no entry at all (top-k of int((1 - s) N) = 0 blocks) still get a
// valid pointer for the attention entry points, which take none as null
// (torch gives an empty tensor a null data pointer); every length is 0 then,
// so the spare element is never read
Tensor csr_entries(const Tensor& like, int64_t nnz) {
  return at::empty({std::max<int64_t>(nnz, 1)}, opts(like, at::kInt));
}

// compact CSR of (start, len, cols) lists: offsets int32 [rows + 1], cols
// int32 [max(nnz, 1)].  One host read of nnz (the allocation size) between the two
// launches.
std::tuple<Tensor, Tensor> lists_to_csr(const Tensor& s_, const Tensor& l_, const Tensor& c_) {
  check_lists(s_, l_, c_);
  TORCH_CHECK(s_.numel() == l_.numel(), "prism.lists_to_csr: start and len differ in length");
  const c10::DeviceGuard guard(s_.device());
  const Tensor s = s_.contiguous(), l = l_.contiguous(), c = c_.contiguous();
  const int64_t rows = s.numel();
  Tensor offsets = at::empty({rows + 1}, opts(s, at::kInt));
  Tensor total = at::empty({1}, opts(s, at::kLong));
  PRISM_TORCH_CALL(prism_lists_csr_offsets, l.data_ptr<int32_t>(), rows, offsets.data_ptr<int32_t>(),
                   total.data_ptr<int64_t>(), stream_of(s));
  const int64_t nnz = total.item<int64_t>();
  TORCH_CHECK_VALUE(nnz <= 2147483647ll, "prism.lists_to_csr: more than 2^31 - 1 list entries (int32 offsets)");
  Tensor out = csr_entries(s, nnz);
  if (nnz > 0)
    PRISM_TORCH_CALL(prism_lists_csr_fill, s.data_ptr<int64_t>(), l.data_ptr<int32_t>(), c.data_ptr<int32_t>(), rows,
                   offsets.data_ptr<int32_t>(), out.data_ptr<int32_t>(), stream_of(s));
  return {offsets, out};
}

// the two halves of lists_to_csr, for callers that batch the host read of
// several lists' nnz: offsets [rows + 1] and the total [1] stay on the device
std::tuple<Tensor, Tensor> lists_csr_offsets(const Tensor& l_) {
  on_gpu(l_, "len");
  check_dtype(l_, at::kInt, "len");
  const c10::DeviceGuard guard(l_.device());
  const Tensor l = l_.contiguous();
  const int64_t rows = l.numel();
  Tensor offsets = at::empty({rows + 1}, opts(l, at::kInt));
  Tensor total = at::empty({1}, opts(l, at::kLong));
  PRISM_TORCH_CALL(prism_lists_csr_offsets, l.data_ptr<int32_t>(), rows, offsets.data_ptr<int32_t>(),
                   total.data_ptr<int64_t>(), stream_of(l));
  return {offsets, total};
}

// entries [nnz] of (start, len, cols) at the offsets of lists_csr_offsets;
// nnz is that call's total (read by the caller)
Tensor lists_csr_fill(const Tensor& s_, const Tensor& l_, const Tensor& c_, const Tensor& offsets_, int64_t nnz) {
  check_lists(s_, l_, c_);
  on_gpu(offsets_, "offsets");
  check_dtype(offsets_, at::kInt, "offsets");
  TORCH_CHECK_VALUE(s_.numel() == l_.numel() && offsets_.numel() == l_.numel() + 1,
                    "prism.lists_csr_fill: start, len and offsets disagree in length");
  TORCH_CHECK_VALUE(nnz >= 0 && nnz <= 2147483647ll, "prism.lists_csr_fill: nnz out of range (int32 offsets)");
  const c10::DeviceGuard guard(s_.device());
  const Tensor s = s_.contiguous(), l = l_.contiguous(), c = c_.contiguous(), offsets = offsets_.contiguous();
  Tensor out = csr_entries(s, nnz);
  if (nnz > 0)
    PRISM_TORCH_CALL(prism_lists_csr_fill, s.data_ptr<int64_t>(), l.data_ptr<int32_t>(), c.data_ptr<int32_t>(),
                     s.numel(), offsets.data_ptr<int32_t>(), out.data_ptr<int32_t>(), stream_of(s));
  return out;
}

Tensor pair_order(const Tensor& ulen_, int64_t group, int64_t tail) {
  on_gpu(ulen_, "ulen");
  check_dtype(ulen_, at::kInt, "ulen");
  const c10::DeviceGuard guard(ulen_.device());
  const Tensor ulen = ulen_.contiguous();
  Tensor order = at::empty({ulen.numel()}, opts(ulen, at::kInt));
  PRISM_TORCH_CALL(prism_pair_order, ulen.data_ptr<int32_t>(), ulen.numel(), (int)group, tail,
                   order.data_ptr<int32_t>(), stream_of(ulen));
  return order;
}

Tensor tile_masks(const Tensor& valid_) {
  on_gpu(valid_, "valid");
  check_dtype(valid_, at::kByte, "valid");
  const c10::DeviceGuard guard(valid_.device());
  const Tensor valid = valid_.contiguous();
  const int64_t Nt = valid.numel() / 64;
  Tensor out = at::empty({Nt}, opts(valid, at::kLong));
  PRISM_TORCH_CALL(prism_tile_masks, valid.data_ptr<uint8_t>(), Nt, (uint64_t*)out.data_ptr<int64_t>(),
                   stream_of(valid));
  return out;
}

Tensor lse_to_m2(const Tensor& lse_) {
  on_gpu(lse_, "lse");
  check_dtype(lse_, at::kFloat, "lse");
  const c10::DeviceGuard guard(lse_.device());
  const Tensor lse = lse_.contiguous();
  Tensor out = at::empty_like(lse);
  PRISM_TORCH_CALL(prism_lse_to_m2, lse.data_ptr<float>(), lse.numel(), out.data_ptr<float>(), stream_of(lse));
  return out;
}

// ------------------------------------------------------------------ attention
struct AttnShape {
  int64_t B, H, Sq, Sk, D;
};
AttnShape attn_shape(const Tensor& q, const Tensor& k, const Tensor& v) {
  on_gpu(q, "q");
  on_gpu(k, "k");
  on_gpu(v, "v");
  check_dtype(q, at::kBFloat16, "q");
  check_dtype(k, at::kBFloat16, "k");
  check_dtype(v, at::kBFloat16, "v");
  TORCH_CHECK_VALUE(q.dim() == 4 && k.dim() == 4 && v.dim() == 4, "prism attention: tensors must be [B,H,S,D]");
  TORCH_CHECK_VALUE(k.sizes() == v.sizes() && k.size(0) == q.size(0) && k.size(1) == q.size(1) && k.size(3) == q.size(3),
                    "prism attention: shapes differ: q ", q.sizes(), ", k ", k.sizes(), ", v ", v.sizes());
  return {q.size(0), q.size(1), q.size(2), k.size(2), q.size(3)};
}
void check_union(const Tensor& us, const Tensor& ul, const Tensor& uc) { check_lists(us, ul, uc); }

// the work-queue counters of one attention launch (persistent workgroups; 8
// int32, one per XCD, zeroed by the entry point on the stream), from the
// caching allocator: each call has its own, and the temporary lives until the
// launch call returns
Tensor work_counter(const Tensor& like) { return at::empty({8}, opts(like, at::kInt)); }

std::tuple<Tensor, Tensor> bsa_fwd(const Tensor& q_, const Tensor& k_, const Tensor& v_, const OptT& masks_,
                                   const Tensor& us_, const Tensor& ul_, const Tensor& uc_, const OptT& pairmap_,
                                   const OptT& order_, double sm_scale) {
  const AttnShape s = attn_shape(q_, k_, v_);
  check_union(us_, ul_, uc_);
  on_gpu(masks_, "tile_masks");
  on_gpu(pairmap_, "pairmap");
  on_gpu(order_, "order");
  const c10::DeviceGuard guard(q_.device());
  const Tensor q = q_.contiguous(), k = k_.contiguous(), v = v_.contiguous();
  const Tensor us = us_.contiguous(), ul = ul_.contiguous(), uc = uc_.contiguous();
  const OptT masks = cont(masks_), pairmap = cont(pairmap_), order = cont(order_);
  Tensor o = at::empty_like(q);
  Tensor lse = at::empty({s.B, s.H, s.Sq}, opts(q, at::kFloat));
  PRISM_TORCH_CALL(prism_bsa_fwd, q.data_ptr(), k.data_ptr(), v.data_ptr(), (int)(s.B * s.H), s.Sq, s.Sk, (int)s.D,
                   (const uint64_t*)p(masks), us.data_ptr<int64_t>(), ul.data_ptr<int32_t>(), uc.data_ptr<int32_t>(),
                   (const int32_t*)p(pairmap), (const int32_t*)p(order), (float)sm_scale, o.data_ptr(),
                   lse.data_ptr<float>(), work_counter(q).data_ptr<int32_t>(), stream_of(q));
  return {o, lse};
}

std::tuple<Tensor, Tensor> bsa_fwd_quad(const Tensor& q_, const Tensor& k_, const Tensor& v_, const OptT& masks_,
                                        const Tensor& us_, const Tensor& ul_, const Tensor& uc_, const OptT& quadmap_,
                                        const OptT& order_, double sm_scale) {
  const AttnShape s = attn_shape(q_, k_, v_);
  check_union(us_, ul_, uc_);
  on_gpu(masks_, "tile_masks");
  on_gpu(quadmap_, "quadmap");
  on_gpu(order_, "order");
  const c10::DeviceGuard guard(q_.device());
  const Tensor q = q_.contiguous(), k = k_.contiguous(), v = v_.contiguous();
  const Tensor us = us_.contiguous(), ul = ul_.contiguous(), uc = uc_.contiguous();
  const OptT masks = cont(masks_), quadmap = cont(quadmap_), order = cont(order_);
  Tensor o = at::empty_like(q);
  Tensor lse = at::empty({s.B, s.H, s.Sq}, opts(q, at::kFloat));
  PRISM_TORCH_CALL(prism_bsa_fwd_quad, q.data_ptr(), k.data_ptr(), v.data_ptr(), (int)(s.B * s.H), s.Sq, s.Sk,
                   (int)s.D, (const uint64_t*)p(masks), us.data_ptr<int64_t>(), ul.data_ptr<int32_t>(),
                   uc.data_ptr<int32_t>(), (const int32_t*)p(quadmap), (const int32_t*)p(order), (float)sm_scale,
                   o.data_ptr(), lse.data_ptr<float>(), work_counter(q).data_ptr<int32_t>(), stream_of(q));
  return {o, lse};
}

Tensor bwd_preprocess(const Tensor& o_, const Tensor& do_) {
  on_gpu(o_, "o");
  on_gpu(do_, "do");
  check_dtype(o_, at::kBFloat16, "o");
  check_dtype(do_, at::kBFloat16, "do");
  TORCH_CHECK_VALUE(o_.sizes() == do_.sizes(), "bwd_preprocess: o and do must have one shape");
  const c10::DeviceGuard guard(o_.device());
  const Tensor o = o_.contiguous(), d = do_.contiguous();
  const int64_t D = o.size(-1);
  Tensor delta = at::empty(o.sizes().slice(0, o.dim() - 1), opts(o, at::kFloat));
  PRISM_TORCH_CALL(prism_bwd_preprocess, o.data_ptr(), d.data_ptr(), o.numel() / D, (int)D, delta.data_ptr<float>(),
                   stream_of(o));
  return delta;
}

std::tuple<Tensor, Tensor> bsa_bwd_dkdv(const Tensor& q_, const Tensor& k_, const Tensor& v_, const Tensor& do_,
                                        const Tensor& m2_, const Tensor& delta_, const OptT& kv_valid_,
                                        const Tensor& us_, const Tensor& ul_, const Tensor& uc_, const OptT& pairmap_,
                                        const OptT& order_, double sm_scale) {
  const AttnShape s = attn_shape(q_, k_, v_);
  check_union(us_, ul_, uc_);
  on_gpu(do_, "do");
  on_gpu(m2_, "m2");
  on_gpu(delta_, "delta");
  on_gpu(kv_valid_, "kv_valid");
  on_gpu(pairmap_, "pairmap");
  on_gpu(order_, "order");
  check_dtype(do_, at::kBFloat16, "do");
  check_dtype(m2_, at::kFloat, "m2");
  check_dtype(delta_, at::kFloat, "delta");
  check_dtype(kv_valid_, at::kByte, "kv_valid");
  TORCH_CHECK_VALUE(do_.sizes() == q_.sizes(), "bsa_bwd_dkdv: do must have q's shape");
  const c10::DeviceGuard guard(q_.device());
  const Tensor q = q_.contiguous(), k = k_.contiguous(), v = v_.contiguous(), d = do_.contiguous();
  const Tensor m2 = m2_.contiguous(), delta = delta_.contiguous();
  const Tensor us = us_.contiguous(), ul = ul_.contiguous(), uc = uc_.contiguous();
  const OptT kv = cont(kv_valid_), pairmap = cont(pairmap_), order = cont(order_);
  Tensor dk = at::empty_like(k), dv = at::empty_like(v);
  PRISM_TORCH_CALL(prism_bsa_bwd_dkdv, q.data_ptr(), k.data_ptr(), v.data_ptr(), d.data_ptr(), m2.data_ptr<float>(),
                   delta.data_ptr<float>(), (int)(s.B * s.H), s.Sq, s.Sk, (int)s.D, (const uint8_t*)p(kv),
                   us.data_ptr<int64_t>(), ul.data_ptr<int32_t>(), uc.data_ptr<int32_t>(), (const int32_t*)p(pairmap),
                   (const int32_t*)p(order), (float)sm_scale, dk.data_ptr(), dv.data_ptr(),
                   work_counter(q).data_ptr<int32_t>(), stream_of(q));
  return {dk, dv};
}

// dQ over pair unions (quad = false) or quad unions (quad = true)
Tensor bsa_bwd_dq_any(const Tensor& q_, const Tensor& k_, const Tensor& v_, const Tensor& do_, const Tensor& m2_,
                      const Tensor& delta_, const OptT& masks_, const Tensor& us_, const Tensor& ul_, const Tensor& uc_,
                      const OptT& pairmap_, const OptT& order_, double sm_scale, bool quad) {
  const AttnShape s = attn_shape(q_, k_, v_);
  check_union(us_, ul_, uc_);
  on_gpu(do_, "do");
  on_gpu(m2_, "m2");
  on_gpu(delta_, "delta");
  on_gpu(masks_, "tile_masks");
  on_gpu(pairmap_, "pairmap");
  on_gpu(order_, "order");
  check_dtype(do_, at::kBFloat16, "do");
  check_dtype(m2_, at::kFloat, "m2");
  check_dtype(delta_, at::kFloat, "delta");
  TORCH_CHECK_VALUE(do_.sizes() == q_.sizes(), "bsa_bwd_dq: do must have q's shape");
  const c10::DeviceGuard guard(q_.device());
  const Tensor q = q_.contiguous(), k = k_.contiguous(), v = v_.contiguous(), d = do_.contiguous();
  const Tensor m2 = m2_.contiguous(), delta = delta_.contiguous();
  const Tensor us = us_.contiguous(), ul = ul_.contiguous(), uc = uc_.contiguous();
  const OptT masks = cont(masks_), pairmap = cont(pairmap_), order = cont(order_);
  Tensor dq = at::empty_like(q);
  auto fn = quad ? &prism_bsa_bwd_dq_quad : &prism_bsa_bwd_dq;
  PRISM_TORCH_CALL(fn, q.data_ptr(), k.data_ptr(), v.data_ptr(), d.data_ptr(), m2.data_ptr<float>(),
                   delta.data_ptr<float>(), (int)(s.B * s.H), s.Sq, s.Sk, (int)s.D, (const uint64_t*)p(masks),
                   us.data_ptr<int64_t>(), ul.data_ptr<int32_t>(), uc.data_ptr<int32_t>(), (const int32_t*)p(pairmap),
                   (const int32_t*)p(order), (float)sm_scale, dq.data_ptr(), work_counter(q).data_ptr<int32_t>(), stream_of(q));
  return dq;
}

Tensor bsa_bwd_dq(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& d, const Tensor& m2,
                  const Tensor& delta, const OptT& masks, const Tensor& us, const Tensor& ul, const Tensor& uc,
                  const OptT& pairmap, const OptT& order, double sm_scale) {
  return bsa_bwd_dq_any(q, k, v, d, m2, delta, masks, us, ul, uc, pairmap, order, sm_scale, false);
}

Tensor bsa_bwd_dq_quad(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& d, const Tensor& m2,
                       const Tensor& delta, const OptT& masks, const Tensor& us, const Tensor& ul, const Tensor& uc,
                       const OptT& quadmap, const OptT& order, double sm_scale) {
  return bsa_bwd_dq_any(q, k, v, d, m2, delta, masks, us, ul, uc, quadmap, order, sm_scale, true);
}

}  // namespace

TORCH_LIBRARY(prism, m) {
  m.def("zone_stats(Tensor v, Tensor? valid, int[] grid, int[] box) -> (Tensor, Tensor)");
  m.def("audio_zone_stats(Tensor norms, Tensor? valid, int[] grid, int[] box) -> (Tensor, Tensor)");
  m.def("zone_gradient(Tensor packed, Tensor axis_valid, int D) -> (Tensor, Tensor)");
  m.def("zone_shapes(Tensor rho_raw, Tensor aniso, Tensor? abar, Tensor? vhat, int method, float lambda_a, "
        "float tau_128, float lambda_128) -> (Tensor, Tensor, Tensor)");
  m.def("assign_shapes(Tensor g, Tensor rho, int method, float tau_128, float lambda_128) -> Tensor");
  m.def("a2v_norms(Tensor residual) -> Tensor");
  m.def("linear_rownorm(Tensor x, Tensor weight, Tensor? bias, int norms_dtype) -> (Tensor, Tensor)");
  m.def("zone_layout(Tensor shape_ids) -> (Tensor, Tensor, Tensor)");
  m.def("rearrange_index(Tensor shape_ids, int[] grid) -> (Tensor, Tensor)");
  m.def("gather_pool(Tensor x, Tensor? valid, Tensor shape_ids, Tensor block_offset, int[] grid, int[] box, int N_b, "
        "bool rows, bool pool, bool counts, Tensor? dot_with) -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)");
  m.def("scatter_rows(Tensor rows, Tensor shape_ids, int[] grid, int[] box, int out_dtype) -> Tensor");
  m.def("chunk_gather_pool(Tensor x, Tensor? valid, int[] grid, int[] pgrid, int[] chunk, int S_out, bool rows, "
        "bool pool, bool counts, Tensor? dot_with) -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)");
  m.def("chunk_scatter_rows(Tensor rows, int[] grid, int[] pgrid, int[] chunk, int out_dtype) -> Tensor");
  m.def("block_scores(Tensor qc, Tensor kc, Tensor? block_count) -> Tensor");
  m.def("select_tiles(Tensor scores, int mode, int k_lo, int ub, float scale, int thr, Tensor block_first_tile, "
        "Tensor? tile_count, int tcap, int bcap, bool want_blocks) -> (Tensor, Tensor, Tensor, Tensor)");
  m.def("tile_rows(Tensor ntiles, Tensor block_id_of_tile, Tensor? q_tile_count, int BH, int Nt, int N_b, "
        "int tcap) -> (Tensor, Tensor)");
  m.def("transpose_lists(Tensor qstart, Tensor qlen, Tensor qcols, int BH, int Ntq, int Ntk) -> (Tensor, Tensor, Tensor)");
  m.def("pair_tiles(Tensor start, Tensor len, Tensor cols, int row_tiles, int col_tiles) -> Tensor");
  m.def("pair_union(Tensor start, Tensor len, Tensor cols, int row_tiles, int col_tiles, Tensor? pairmap, "
        "Tensor? tile_masks) -> (Tensor, Tensor, Tensor)");
  m.def("quad_union(Tensor start, Tensor len, Tensor cols, int row_tiles, int col_tiles, Tensor? pairmap, "
        "Tensor? tile_masks) -> (Tensor, Tensor, Tensor)");
  m.def("pair_order(Tensor ulen, int group, int tail) -> Tensor");
  m.def("lists_to_csr(Tensor start, Tensor len, Tensor cols) -> (Tensor, Tensor)");
  m.def("lists_csr_offsets(Tensor len) -> (Tensor, Tensor)");
  m.def("lists_csr_fill(Tensor start, Tensor len, Tensor cols, Tensor offsets, int nnz) -> Tensor");
  m.def("tile_masks(Tensor valid) -> Tensor");
  m.def("lse_to_m2(Tensor lse) -> Tensor");
  m.def("bsa_fwd(Tensor q, Tensor k, Tensor v, Tensor? tile_masks, Tensor ustart, Tensor ulen, Tensor ucols, "
        "Tensor? pairmap, Tensor? order, float sm_scale) -> (Tensor, Tensor)");
  m.def("bsa_fwd_quad(Tensor q, Tensor k, Tensor v, Tensor? tile_masks, Tensor ustart, Tensor ulen, Tensor ucols, "
        "Tensor? quadmap, Tensor? order, float sm_scale) -> (Tensor, Tensor)");
  m.def("bwd_preprocess(Tensor o, Tensor do) -> Tensor");
  m.def("bsa_bwd_dkdv(Tensor q, Tensor k, Tensor v, Tensor do, Tensor m2, Tensor delta, Tensor? kv_valid, "
        "Tensor ustart, Tensor ulen, Tensor ucols, Tensor? pairmap, Tensor? order, float sm_scale) -> (Tensor, Tensor)");
  m.def("bsa_bwd_dq(Tensor q, Tensor k, Tensor v, Tensor do, Tensor m2, Tensor delta, Tensor? tile_masks, "
        "Tensor ustart, Tensor ulen, Tensor ucols, Tensor? pairmap, Tensor? order, float sm_scale) -> Tensor");
  m.def("bsa_bwd_dq_quad(Tensor q, Tensor k, Tensor v, Tensor do, Tensor m2, Tensor delta, Tensor? tile_masks, "
        "Tensor ustart, Tensor ulen, Tensor ucols, Tensor? quadmap, Tensor? order, float sm_scale) -> Tensor");
}

// GPU tensors of the ROCm build dispatch under torch's CUDA key
TORCH_LIBRARY_IMPL(prism, CUDA, m) {
  m.impl("zone_stats", &zone_stats);
  m.impl("audio_zone_stats", &audio_zone_stats);
  m.impl("zone_gradient", &zone_gradient);
  m.impl("zone_shapes", &zone_shapes);
  m.impl("assign_shapes", &assign_shapes);
  m.impl("a2v_norms", &a2v_norms);
  m.impl("linear_rownorm", &linear_rownorm);
  m.impl("zone_layout", &zone_layout);
  m.impl("rearrange_index", &rearrange_index);
  m.impl("gather_pool", &gather_pool);
  m.impl("scatter_rows", &scatter_rows);
  m.impl("chunk_gather_pool", &chunk_gather_pool);
  m.impl("chunk_scatter_rows", &chunk_scatter_rows);
  m.impl("block_scores", &block_scores);
  m.impl("select_tiles", &select_tiles);
  m.impl("tile_rows", &tile_rows);
  m.impl("transpose_lists", &transpose_lists);
  m.impl("pair_tiles", &pair_tiles);
  m.impl("pair_union", &pair_union);
  m.impl("quad_union", &quad_union);
  m.impl("pair_order", &pair_order);
  m.impl("lists_to_csr", &lists_to_csr);
  m.impl("lists_csr_offsets", &lists_csr_offsets);
  m.impl("lists_csr_fill", &lists_csr_fill);
  m.impl("tile_masks", &tile_masks);
  m.impl("lse_to_m2", &lse_to_m2);
  m.impl("bsa_fwd", &bsa_fwd);
  m.impl("bsa_fwd_quad", &bsa_fwd_quad);
  m.impl("bwd_preprocess", &bwd_preprocess);
  m.impl("bsa_bwd_dkdv", &bsa_bwd_dkdv);
  m.impl("bsa_bwd_dq", &bsa_bwd_dq);
  m.impl("bsa_bwd_dq_quad", &bsa_bwd_dq_quad);
}
