// Gating / selection path of the Polynomial Mixer for gfx950.
//
// Forward (pom/pom.py:207 + :103-122, with RoPE pom/pom_rope.py:522-525):
//   z  = y_s + se_bias
//   s  = hardsigmoid(z)                       (relu6(z + 3) / 6)
//   s' = R(pos_query) s                       (RoPE variants only)
//   sh = s' * hagg[b, group(token)]           (hagg in the element type)
// One streaming pass: reads y_s, writes sh; everything in between stays in
// registers (the reference makes three passes: add, hardsigmoid, multiply).
//
// Backward:
//   d s' = dsh * hagg,  ds = R^T d s',  dz = ds * hardsigmoid'(z)  -> dY_s (strided)
//   dhagg[b, g] = sum_{tokens of g} dsh * s'                        (fp32)
//   dbias       = sum_{all tokens} dz                               (fp32)
// Reductions use the chunk decomposition of the aggregation kernels: chunk
// partials, then one finalize kernel that sums them in a fixed order.
#pragma once

#include "agg_impl.h"

namespace pom {

template <typename T, int CPT, int MODE, bool TR>
__global__ void __launch_bounds__(kThreads) gate_fwd_kernel(const GateParams p, int per_token) {
  using Map = LaneMap<CPT, MODE>;
  constexpr int CPT2 = Map::CPT2;
  constexpr bool ROPE = Mode_<MODE>::rope;
  constexpr int U = ROPE ? 4 : 8;

  const LaneGeom G(p.g.lpr_log2);
  const int64_t slab = blockIdx.x, chunk = blockIdx.y, b = blockIdx.z;
  int64_t f, rbeg, rend;
  chunk_rows(p.g, chunk, p.N, f, rbeg, rend);
  const int64_t vcol = slab * G.lpr + G.lcol;
  // Lanes past the channels run the walk on channel 0 (every wave takes part
  // in the staged channel-major stores) and store nothing.
  const bool active = vcol < p.g.nvec;
  Map map;
  map.init(active ? vcol : 0, p.P);
  const int64_t ngroups = per_token ? p.N : p.g.F;

  float bias[CPT2], hv[CPT2];
  if (p.bias.ptr) {
    param_gather<CPT2>(p.bias, [&](int i) { return map.chan(i); }, bias);
  } else {
#pragma unroll
    for (int i = 0; i < CPT2; ++i) bias[i] = 0.0f;
  }
  const T* hb = reinterpret_cast<const T*>(p.hagg) + b * ngroups * p.P;
  if (!per_token) {
    Pack<T, CPT> h1, h2;
    h1.load(hb + f * p.P + map.c1);
    if constexpr (ROPE) h2.load(hb + f * p.P + map.c2);
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      hv[i] = h1.get(i);
      if constexpr (ROPE) hv[CPT + i] = h2.get(i);
    }
  }

  const T* yb = reinterpret_cast<const T*>(p.ys) + b * p.ysb;
  T* ob = reinterpret_cast<T*>(p.sh) + b * p.shb;
  const RowWalk W = TR ? RowWalk::consecutive(rbeg, rend, G.wave * G.rpw + G.lrow, G.rs, U)
                       : RowWalk(rbeg, rend, G.wave * G.rpw + G.lrow, G.rs, U);
  __shared__ __attribute__((aligned(16))) unsigned char tile_raw[TR ? TrTile<U, CPT2>::kElems * sizeof(T) : 16];
  T* tile = reinterpret_cast<T*>(tile_raw);

  struct Buf {
    Pack<T, CPT> y1[U], y2[ROPE ? U : 1];
  };
  auto load = [&](Buf& bf, int64_t base, bool clamp) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const T* row = yb + W.row(base, u, clamp) * p.ysn;
      bf.y1[u].load_stream(row + map.c1);
      if constexpr (ROPE) bf.y2[u].load_stream(row + map.c2);
    }
  };
  auto step = [&](const Buf& bf, int64_t base, auto tail_tag) {
    constexpr bool TAIL = decltype(tail_tag)::value;
    float ot[TR ? U : 1][CPT2];
    const auto& y1 = bf.y1;
    const auto& y2 = bf.y2;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t n = W.row(base, u, TAIL);
      if (per_token) {
        Pack<T, CPT> h1, h2;
        h1.load(hb + n * p.P + map.c1);
        if constexpr (ROPE) h2.load(hb + n * p.P + map.c2);
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
          hv[i] = h1.get(i);
          if constexpr (ROPE) hv[CPT + i] = h2.get(i);
        }
      }
      float o1[CPT], o2[CPT];
      T* orow = ob + n * p.shn;
      if constexpr (ROPE) {
        float cs[CPT], sn[CPT];
        load_table<CPT>(p.rope, map.table, n, map.tcol, cs, sn);
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
          const float a = hsig(y1[u].get(i) + bias[i]), bb = hsig(y2[u].get(i) + bias[CPT + i]);
          o1[i] = (a * cs[i] - bb * sn[i]) * hv[i];
          o2[i] = (bb * cs[i] + a * sn[i]) * hv[CPT + i];
        }
        if (active && (!TAIL || W.valid(base, u))) {
          VecIO<T, CPT>::store(orow + map.c1, o1);
          VecIO<T, CPT>::store(orow + map.c2, o2);
        }
        if constexpr (TR) {
#pragma unroll
          for (int i = 0; i < CPT; ++i) {
            ot[u][i] = o1[i];
            ot[u][CPT + i] = o2[i];
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < CPT; ++i) o1[i] = hsig(y1[u].get(i) + bias[i]) * hv[i];
        if (active && (!TAIL || W.valid(base, u))) VecIO<T, CPT>::store(orow + map.c1, o1);
        if constexpr (TR) {
#pragma unroll
          for (int i = 0; i < CPT; ++i) ot[u][i] = o1[i];
        }
      }
    }
    if constexpr (TR) {
      const int64_t left = W.nrows - base;
      store_tr_staged<T, U, CPT2>(
          p.sht, G, b, W.rbeg + base, left < W.step ? left : W.step,
          [&](int l, int i) { return slab_chan<CPT, MODE>(slab, G.lpr, p.g.nvec, p.P, l, i); }, ot, tile);
    }
  };
  walk_rows<Buf>(W, load, step);
}

template <typename T, int CPT, int MODE, bool TR>
__global__ void __launch_bounds__(kThreads) gate_bwd_kernel(const GateParams p, int per_token) {
  using Map = LaneMap<CPT, MODE>;
  constexpr int CPT2 = Map::CPT2;
  constexpr bool ROPE = Mode_<MODE>::rope;
  constexpr int U = ROPE ? 2 : 4;
  __shared__ float red[kWaves][kMaxLpr * CPT2];

  const LaneGeom G(p.g.lpr_log2);
  const int64_t slab = blockIdx.x, chunk = blockIdx.y, b = blockIdx.z;
  int64_t f, rbeg, rend;
  chunk_rows(p.g, chunk, p.N, f, rbeg, rend);
  const int64_t vcol = slab * G.lpr + G.lcol;
  const bool active = vcol < p.g.nvec;
  Map map;
  map.init(active ? vcol : 0, p.P);
  const int64_t ngroups = per_token ? p.N : p.g.F;

  float bias[CPT2], hv[CPT2], dh[CPT2], db[CPT2];
  const T* hb = reinterpret_cast<const T*>(p.hagg) + b * ngroups * p.P;
  if (p.bias.ptr) {
    param_gather<CPT2>(p.bias, [&](int i) { return map.chan(i); }, bias);
  } else {
#pragma unroll
    for (int i = 0; i < CPT2; ++i) bias[i] = 0.0f;
  }
  {
    T raw[CPT2];
#pragma unroll
    for (int i = 0; i < CPT2; ++i) raw[i] = hb[(per_token ? 0 : f) * p.P + map.chan(i)];
#pragma unroll
    for (int i = 0; i < CPT2; ++i) {
      bias[i] = active ? bias[i] : 0.0f;
      hv[i] = (active && !per_token) ? to_f32<T>(raw[i]) : 0.0f;
      dh[i] = 0.0f;
      db[i] = 0.0f;
    }
  }

  const T* yb = reinterpret_cast<const T*>(p.ys) + b * p.ysb;
  const T* gb = reinterpret_cast<const T*>(p.dsh) + b * p.dsb;
  T* dyb = reinterpret_cast<T*>(p.dys) + b * p.dyb;
  const RowWalk W = TR ? RowWalk::consecutive(rbeg, rend, G.wave * G.rpw + G.lrow, G.rs, U)
                       : RowWalk(rbeg, rend, G.wave * G.rpw + G.lrow, G.rs, U);
  __shared__ __attribute__((aligned(16))) unsigned char tile_raw[TR ? TrTile<U, CPT2>::kElems * sizeof(T) : 16];
  T* tile = reinterpret_cast<T*>(tile_raw);

  struct Buf {
    Pack<T, CPT> y1[U], y2[ROPE ? U : 1], g1[U], g2[ROPE ? U : 1];
  };
  auto load = [&](Buf& bf, int64_t base, bool clamp) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t rr = W.row(base, u, clamp);
      const T* yrow = yb + rr * p.ysn;
      const T* grow = gb + rr * p.dsn;
      bf.y1[u].load_stream(yrow + map.c1);
      bf.g1[u].load_stream(grow + map.c1);
      if constexpr (ROPE) {
        bf.y2[u].load_stream(yrow + map.c2);
        bf.g2[u].load_stream(grow + map.c2);
      }
    }
  };
  auto step = [&](const Buf& bf, int64_t base, auto tail_tag) {
    constexpr bool TAIL = decltype(tail_tag)::value;
    float dt[TR ? U : 1][CPT2];
    const auto& y1 = bf.y1;
    const auto& y2 = bf.y2;
    const auto& g1 = bf.g1;
    const auto& g2 = bf.g2;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool in = !TAIL || W.valid(base, u);
      const int64_t n = W.row(base, u, TAIL);
      if (per_token) {
#pragma unroll
        for (int i = 0; i < CPT2; ++i) hv[i] = to_f32<T>(hb[n * p.P + map.chan(i)]);
      }
      float z[CPT2], s[CPT2], gv[CPT2];
#pragma unroll
      for (int i = 0; i < CPT; ++i) {
        z[i] = y1[u].get(i) + bias[i];
        gv[i] = TAIL ? (in ? g1[u].get(i) : 0.0f) : g1[u].get(i);
        if constexpr (ROPE) {
          z[CPT + i] = y2[u].get(i) + bias[CPT + i];
          gv[CPT + i] = TAIL ? (in ? g2[u].get(i) : 0.0f) : g2[u].get(i);
        }
      }
#pragma unroll
      for (int i = 0; i < CPT2; ++i) s[i] = hsig(z[i]);
      float dcon[CPT2], ds[CPT2];
      if constexpr (ROPE) {
        float cs[CPT], sn[CPT];
        load_table<CPT>(p.rope, map.table, n, map.tcol, cs, sn);
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
          const float a = s[i], bb = s[CPT + i];
          const float d1 = gv[i] * hv[i], d2 = gv[CPT + i] * hv[CPT + i];   // d (rotated gate)
          dcon[i] = gv[i] * (a * cs[i] - bb * sn[i]);
          dcon[CPT + i] = gv[CPT + i] * (bb * cs[i] + a * sn[i]);
          ds[i] = d1 * cs[i] + d2 * sn[i];
          ds[CPT + i] = d2 * cs[i] - d1 * sn[i];
        }
      } else {
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
          dcon[i] = gv[i] * s[i];
          ds[i] = gv[i] * hv[i];
        }
      }
      float dz[CPT2];
#pragma unroll
      for (int i = 0; i < CPT2; ++i) {
        dz[i] = ds[i] * hsig_grad(z[i]);
        db[i] += dz[i];
        if constexpr (TR) dt[u][i] = dz[i];
      }
      if (per_token) {
        // one token per group: the gradient of hagg is the contribution itself
        if (active && in) {
          float* drow = p.dhagg + (b * p.N + n) * p.P;
          float t[CPT];
#pragma unroll
          for (int i = 0; i < CPT; ++i) t[i] = dcon[i];
          store_f32<CPT>(drow + map.c1, t);
          if constexpr (ROPE) {
#pragma unroll
            for (int i = 0; i < CPT; ++i) t[i] = dcon[CPT + i];
            store_f32<CPT>(drow + map.c2, t);
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < CPT2; ++i) dh[i] += dcon[i];
      }
      if (active && in) {
        T* drow = dyb + n * p.dyn;
        float t[CPT];
#pragma unroll
        for (int i = 0; i < CPT; ++i) t[i] = dz[i];
        VecIO<T, CPT>::store(drow + map.c1, t);
        if constexpr (ROPE) {
#pragma unroll
          for (int i = 0; i < CPT; ++i) t[i] = dz[CPT + i];
          VecIO<T, CPT>::store(drow + map.c2, t);
        }
      }
    }
    if constexpr (TR) {
      const int64_t left = W.nrows - base;
      store_tr_staged<T, U, CPT2>(
          p.dyst, G, b, W.rbeg + base, left < W.step ? left : W.step,
          [&](int l, int i) { return slab_chan<CPT, MODE>(slab, G.lpr, p.g.nvec, p.P, l, i); }, dt, tile);
    }
  };
  // every lane walks (lanes past the channels on channel 0, storing nothing):
  // the staged channel-major stores synchronise the workgroup
  walk_rows<Buf>(W, load, step);

  // Chunk partials: dhagg (unless per-token) and dbias.
  const int nslot = G.lpr * CPT2;
  const int64_t prow = (b * p.g.nch + chunk) * p.P;
  for (int pass = per_token ? 1 : 0; pass < 2; ++pass) {
    if (pass == 1 && !p.dbias.ptr) break;
    float* dst = pass == 0 ? p.part_h : p.part_b;
#pragma unroll
    for (int i = 0; i < CPT2; ++i) {
      const float v = xor_sum_rows(pass == 0 ? dh[i] : db[i], G.lb);
      if (G.lrow == 0) red[G.wave][G.lcol * CPT2 + i] = v;
    }
    __syncthreads();
    for (int s = G.tid; s < nslot; s += kThreads) {
      const int l = s / CPT2, i = s - l * CPT2;
      const int64_t vc = slab * G.lpr + l;
      if (vc >= p.g.nvec) continue;
      float v = 0.0f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) v += red[w][s];
      Map m2;
      m2.init(vc, p.P);
      dst[prow + m2.chan(i)] = v;
    }
    __syncthreads();
  }
}

// dhagg[b, g, c] = sum of the group's chunk partials; dbias[c] = sum over all.
static __global__ void __launch_bounds__(kThreads) gate_bwd_finalize(const GateParams p, int per_token) {
  const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int64_t nch = p.g.nch, cpf = p.g.cpf;
  if (!per_token && idx < p.B * p.P) {
    const int64_t b = idx / p.P, c = idx - b * p.P;
    constexpr int FB = 8;   // frames whose chunk loads are issued together
    for (int64_t f0 = 0; f0 < p.g.F; f0 += FB) {
      float sf[FB];
#pragma unroll
      for (int q = 0; q < FB; ++q) sf[q] = 0.0f;
      for (int64_t k = 0; k < cpf; ++k) {   // each frame's chunks summed in chunk order
        float v[FB];
#pragma unroll
        for (int q = 0; q < FB; ++q)
          v[q] = f0 + q < p.g.F ? p.part_h[(b * nch + (f0 + q) * cpf + k) * p.P + c] : 0.0f;
#pragma unroll
        for (int q = 0; q < FB; ++q) sf[q] += v[q];
      }
#pragma unroll
      for (int q = 0; q < FB; ++q)
        if (f0 + q < p.g.F) p.dhagg[(b * p.g.F + f0 + q) * p.P + c] = sf[q];
    }
  }
  if (p.dbias.ptr && idx < p.P) {
    const int64_t rows = p.B * nch;
    float s = 0.0f;
    int64_t r = 0;
    for (; r + 16 <= rows; r += 16) {   // sixteen loads in flight, summed in row order
      float v[16];
#pragma unroll
      for (int q = 0; q < 16; ++q) v[q] = p.part_b[(r + q) * p.P + idx];
#pragma unroll
      for (int q = 0; q < 16; ++q) s += v[q];
    }
    for (; r < rows; ++r) s += p.part_b[r * p.P + idx];
    param_set(p.dbias, idx, s);
  }
}

template <typename T, int CPT, bool TR>
hipError_t gate_fwd_tr(const GateParams& p, hipStream_t st, int per_token) {
  const dim3 grid((unsigned)p.g.nslabs, (unsigned)p.g.nch, (unsigned)p.B), block(kThreads);
  switch (p.mode) {
    case MODE_PLAIN: hipLaunchKernelGGL((gate_fwd_kernel<T, CPT, MODE_PLAIN, TR>), grid, block, 0, st, p, per_token); break;
    case MODE_ROPE1D: hipLaunchKernelGGL((gate_fwd_kernel<T, CPT, MODE_ROPE1D, TR>), grid, block, 0, st, p, per_token); break;
    case MODE_ROPE2D: hipLaunchKernelGGL((gate_fwd_kernel<T, CPT, MODE_ROPE2D, TR>), grid, block, 0, st, p, per_token); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename T, int CPT>
hipError_t gate_fwd_cpt(const GateParams& p, hipStream_t st, int per_token) {
  if constexpr (kTrBuilt<T, CPT>) {
    if (p.sht.data) return gate_fwd_tr<T, CPT, true>(p, st, per_token);
  } else {
    if (p.sht.data) return hipErrorInvalidValue;
  }
  return gate_fwd_tr<T, CPT, false>(p, st, per_token);
}

template <typename T, int CPT, bool TR>
hipError_t gate_bwd_tr(const GateParams& p, hipStream_t st, int per_token) {
  const dim3 grid((unsigned)p.g.nslabs, (unsigned)p.g.nch, (unsigned)p.B), block(kThreads);
  switch (p.mode) {
    case MODE_PLAIN: hipLaunchKernelGGL((gate_bwd_kernel<T, CPT, MODE_PLAIN, TR>), grid, block, 0, st, p, per_token); break;
    case MODE_ROPE1D: hipLaunchKernelGGL((gate_bwd_kernel<T, CPT, MODE_ROPE1D, TR>), grid, block, 0, st, p, per_token); break;
    case MODE_ROPE2D: hipLaunchKernelGGL((gate_bwd_kernel<T, CPT, MODE_ROPE2D, TR>), grid, block, 0, st, p, per_token); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename T, int CPT>
hipError_t gate_bwd_cpt(const GateParams& p, hipStream_t st, int per_token) {
  if constexpr (kTrBuilt<T, CPT>) {
    if (p.dyst.data) return gate_bwd_tr<T, CPT, true>(p, st, per_token);
  } else {
    if (p.dyst.data) return hipErrorInvalidValue;
  }
  return gate_bwd_tr<T, CPT, false>(p, st, per_token);
}

// per_token: hagg holds one row per token (token-causal aggregation).
template <typename T>
hipError_t gate_fwd_t(const GateParams& p, int per_token, hipStream_t st) {
  POM_CPT_SWITCH(T, p.g.cpt, gate_fwd_cpt, p, st, per_token)
}

template <typename T>
hipError_t gate_bwd_t(const GateParams& p, int per_token, hipStream_t st) {
  hipError_t e;
  {
    auto run = [&]() -> hipError_t { POM_CPT_SWITCH(T, p.g.cpt, gate_bwd_cpt, p, st, per_token) };
    e = run();
  }
  if (e != hipSuccess) return e;
  const int64_t n = per_token ? p.P : (p.B * p.P > p.P ? p.B * p.P : p.P);
  hipLaunchKernelGGL(gate_bwd_finalize, flat_grid(n), dim3(kThreads), 0, st, p, per_token);
  return hipGetLastError();
}

}  // namespace pom
