// decode.hip - BD3-LM decode attention over the KV cache for gfx950.
//
// Counterpart of block_sparse_decode_kern (kernels/BlockSparseDecodeAttention.py:40-110)
// and split_kv_kern / split_kv_reduce_kern (kernels/SplitKVDecodeAttention.py:16-127).
// Queries are the last q_len of kv_len positions; row i sees key j iff
// j / bs <= (kv_len - q_len + i) / bs and j < kv_len (bd3_mask.h).
//
// decode_partial: one workgroup per (split, 32-row query tile, batch*head).
//   The split's key range is cut into 32-key chunks that the waves (four, or
//   eight when the grid has fewer workgroups than CUs and a split holds at
//   least 16 chunks) take in turn; each wave runs an online softmax over its
//   chunks, then the waves' states are merged through LDS. With one split the workgroup writes O
//   directly; otherwise it writes a normalised fp32 partial and its log2-LSE.
//   K and V are read once per call, with non-temporal loads (ld16_stream) so
//   the stream does not evict other data from L2 / MALL; measured 7% faster
//   than cached loads at the configs[3] shape. Each load instruction fetches
//   8 whole 128-byte key rows (8 lanes per row) into registers; the rows go
//   to the wave's private row-major K and V tiles in LDS, and the loads of
//   the wave's next chunk are issued before the current one is computed.
//   S^T (32 keys x 32 rows) = K Q^T on v_mfma_f32_32x32x16_bf16 with K rows
//   read from the K tile as A operands; V is read transposed
//   (ds_read_b64_tr_b16) as the A operand of O^T += V^T P^T.
// decode16_partial: the same for q_len <= 16 (a cached denoising step of one
//   16-token block) on v_mfma_f32_16x16x32_bf16, so no MFMA row or softmax
//   lane is spent on absent queries. Waves step over 32-key chunks fetched
//   with full-row loads into registers, staged through wave-private LDS
//   tiles; the loads of a wave's next chunk are in flight while the current
//   one is computed. When one workgroup per split would overfill the GPU, a
//   workgroup takes several consecutive splits (splits_per_group): its waves
//   deal the chunks of all of them out continuously and merge each split's
//   share into their running state at the split's end (the same LSE merge
//   the combine pass applies), so the result equals one partial per split
//   merged, with fewer partials in memory (none when one workgroup covers
//   all of a head's splits).
// decode_combine: merges the splits, weights exp2(lse_s - max lse) (the
//   reference's split_kv_reduce_kern arithmetic, :109-127), 4 outputs per
//   thread.
#include "bd3_device.h"
#include "bd3_launch.h"
#include "bd3_mask.h"

namespace bd3 {
namespace {

constexpr int kNW = 4;
constexpr int kThreads = kNW * 64;

constexpr int kQT = 32;       // query rows per workgroup
constexpr int kSub = 32;      // keys per wave step
constexpr int kStride = 72;   // padded LDS row (bf16)
constexpr int kVElems = 2 * kSub * kStride;  // a wave's K and V tiles

template <int NW>
struct MergeLds {
  float o[NW][kHeadDim][kQT + 1];  // O^T per wave (unnormalised), padded
  float m[NW][kQT];
  float l[NW][kQT];
};
template <int NW>
constexpr size_t partial_smem_bytes() {
  constexpr size_t v = sizeof(__bf16) * NW * kVElems;
  return v > sizeof(MergeLds<NW>) ? v : sizeof(MergeLds<NW>);
}

// NW waves share the key chunks of one (split, 32-row tile, batch*head).
template <int NW>
__global__ __launch_bounds__(NW * 64) void decode_partial(DecodeArgs a) {
  constexpr int kNW = NW;
  constexpr int kThreads = NW * 64;
  __shared__ __attribute__((aligned(16))) char smem[partial_smem_bytes<NW>()];
  __bf16* ks = reinterpret_cast<__bf16*>(smem) + (wi_x() >> 6) * 2 * kSub * kStride;
  __bf16* vs = ks + kSub * kStride;

  const int tid = wi_x();
  const int lane = tid & 63;
  const int wave = wave_uniform(tid >> 6);
  const int l32 = lane & 31;
  const int g = lane >> 5;

  const int split = wg_x();
  const int qt = wg_y();
  const int bh = wg_z();
  const int b = bh / a.heads, h = bh - b * a.heads;
  const int i0 = qt * kQT;

  const uint16_t* qp = a.q + b * a.sq.b + h * a.sq.h;
  const uint16_t* kp = a.k + b * a.sk.b + h * a.sk.h;
  const uint16_t* vp = a.v + b * a.sv.b + h * a.sv.h;

  // Q^T B operand: lane holds row i0 + l32 (clamped), d = 16c + 8g .. +7.
  const int myi = i0 + l32;
  const int qrow = imin(myi, a.q_len - 1);
  bf16x8 qreg[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
    qreg[c] = __builtin_bit_cast(bf16x8, ld16(qp + (int64_t)qrow * a.sq.s + 16 * c + 8 * g));
  // Row i sees keys [0, khi).
  const int pos = a.kv_len - a.q_len + myi;
  const int khi = imin((pos / a.bs + 1) * a.bs, a.kv_len);

  const int key_end = decode_key_end(i0, kQT, a.q_len, a.kv_len, a.bs);
  const int lo = split * a.split_len;
  const int hi = imin(lo + a.split_len, key_end);
  const int n_chunks = hi > lo ? (hi - lo + kSub - 1) / kSub : 0;

  f32x16 oacc[2] = {};
  float m = -INFINITY, lsum = 0.f;

  // 32-key chunks, full-row loads, next chunk in flight during the compute and
  // a per-head start rotation: the read order of decode16_partial.
  const int r0 = n_chunks > 0 ? (bh * 7) % n_chunks : 0;
  auto rot = [&](int i) { const int c = i + r0; return c >= n_chunks ? c - n_chunks : c; };
  u32x4 kr[4], vr[4];  // lane + 64j -> key row c0 + lane/8 + 8j, 16-byte part lane%8
  auto load = [&](int ch) {
    const int c0 = lo + rot(ch) * kSub;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int key = imin(c0 + (lane >> 3) + 8 * j, a.kv_len - 1);
      kr[j] = ld16_stream(kp + (int64_t)key * a.sk.s + 8 * (lane & 7));
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int key = imin(c0 + (lane >> 3) + 8 * j, a.kv_len - 1);
      vr[j] = ld16_stream(vp + (int64_t)key * a.sv.s + 8 * (lane & 7));
    }
  };
  if (wave < n_chunks) load(wave);
  const int tr_row = (lane & 15) >> 2;
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

  for (int ch = wave; ch < n_chunks; ch += kNW) {
    const int c0 = lo + rot(ch) * kSub;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int off = ((lane >> 3) + 8 * j) * kStride + 8 * (lane & 7);
      *reinterpret_cast<u32x4*>(&ks[off]) = kr[j];
      *reinterpret_cast<u32x4*>(&vs[off]) = vr[j];
    }
    if (ch + kNW < n_chunks) load(ch + kNW);

    // keys past hi belong to the next split (or are invisible)
    int cls = c0 >= hi ? kNone : decode_class(i0, kQT, c0, kSub, a.q_len, a.kv_len, a.bs);
    if (cls == kFull && c0 + kSub > hi) cls = kPartial;
    if (cls == kNone) continue;
    // S^T (32 keys x 32 rows): A = K rows from the tile (lane: key l32, d 16c + 8g .. +7).
    f32x16 s = {};
#pragma unroll
    for (int c = 0; c < 4; ++c)
      s = mfma32(*reinterpret_cast<const bf16x8*>(&ks[l32 * kStride + 16 * c + 8 * g]), qreg[c], s);
    if (cls == kPartial) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = c0 + 8 * (r >> 2) + 4 * g + (r & 3);
        s[r] = (key < khi && key < hi) ? s[r] : -INFINITY;
      }
    }

    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[r]);
    mx = max_xor32(mx);
    const float m_new = fmaxf(m, mx * a.scale_log2);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = fast_exp2(m - m_use);
    m = m_new;
    lsum *= alpha;
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;

    float p[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      p[r] = fast_exp2(fmaf(s[r], a.scale_log2, -m_use));
      lsum += p[r];
    }
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      const bf16x8 pop = to_bf16x8(p[8 * kc], p[8 * kc + 1], p[8 * kc + 2], p[8 * kc + 3],
                                   p[8 * kc + 4], p[8 * kc + 5], p[8 * kc + 6], p[8 * kc + 7]);
      const int row = 16 * kc + 4 * g + tr_row;
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        const bf16x8 va = cat8(lds_read_tr(&vs[row * kStride + 32 * db + tr_col]),
                               lds_read_tr(&vs[(row + 8) * kStride + 32 * db + tr_col]));
        oacc[db] = mfma32(va, pop, oacc[db]);
      }
    }
  }

  // Merge the four waves' states.
  lsum = sum_xor32(lsum);
  __syncthreads();  // V staging area is reused below
  MergeLds<NW>* ml = reinterpret_cast<MergeLds<NW>*>(smem);
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int d = 32 * db + 8 * (r >> 2) + 4 * g + (r & 3);
      ml->o[wave][d][l32] = oacc[db][r];
    }
  if (g == 0) {
    ml->m[wave][l32] = m;
    ml->l[wave][l32] = lsum;
  }
  __syncthreads();

  const int split_out = a.groups > 1;
  uint16_t* op = a.o + b * a.so.b + h * a.so.h;
  const int64_t slot = ((int64_t)bh * a.q_tiles + qt) * a.groups + split;
#pragma unroll
  for (int j = 0; j < (kQT * kHeadDim) / kThreads; ++j) {
    const int e = tid + kThreads * j;
    const int row = e >> 6, d = e & 63;
    float mm = -INFINITY;
#pragma unroll
    for (int w = 0; w < kNW; ++w) mm = fmaxf(mm, ml->m[w][row]);
    const float mu = (mm == -INFINITY) ? 0.f : mm;
    float lt = 0.f, ot = 0.f;
#pragma unroll
    for (int w = 0; w < kNW; ++w) {
      const float wgt = fast_exp2(ml->m[w][row] - mu);
      lt += wgt * ml->l[w][row];
      ot += wgt * ml->o[w][d][row];
    }
    if (!split_out) {
      if (i0 + row < a.q_len) {
        const __bf16 y = (__bf16)(ot / lt);
        op[(int64_t)(i0 + row) * a.so.s + d] = __builtin_bit_cast(uint16_t, y);
      }
    } else {
      a.part_o[(slot * kQT + row) * kHeadDim + d] = lt > 0.f ? ot / lt : 0.f;
      if (d == 0) a.part_lse[slot * kQT + row] = lt > 0.f ? mm + fast_log2(lt) : -INFINITY;
    }
  }
}

// ---------------------------------------------------------------------------
// q_len <= 16: 16-row query tile on v_mfma_f32_16x16x32_bf16, 32-key chunks.
//   K and V of a chunk are fetched with full-row loads (8 lanes x 16 bytes
//   cover one 128-byte key row, so every load instruction requests 8 whole
//   rows): measured on MI355X, half-row requests (16 keys x 64 bytes per
//   instruction, the layout the MFMA operands want) cost 7-12% of the HBM
//   read rate at this access pattern, and 32-key chunks (8 KB of K and V in
//   flight per wave) stream 7% faster than 64-key chunks. Both tiles go
//   through the wave's private row-major LDS tiles:
//   S^T block (16 keys x 16 rows) = K Q^T: A = K read from the K tile (lane:
//   key 16kb + lane%16, d 32c + 8h .. +7 with h = lane/16), B = Q^T (lane:
//   row lane%16, same d); result lane (row lane%16, h) holds keys
//   16kb + 4h + r.
//   O^T (16 d x 16 rows) += V^T P^T over the 32 keys: B = P^T from the S^T
//   registers of both key blocks, A = V^T read transposed from the V tile
//   with the same key order.
constexpr int kQ16 = 16;
constexpr int kChunk16 = 32;                         // keys per wave step
constexpr int kTile16 = kChunk16 * kStride;          // bf16 per K or V tile
constexpr int kLoads16 = kChunk16 * 128 / (64 * 16);  // 16-byte loads per lane and tensor

template <int NW>
struct Merge16 {
  float o[NW][kHeadDim][kQ16 + 1];
  float m[NW][kQ16];
  float l[NW][kQ16];
};
template <int NW>
constexpr size_t smem16_bytes() {
  return sizeof(__bf16) * NW * 2 * kTile16 > sizeof(Merge16<NW>) ? sizeof(__bf16) * NW * 2 * kTile16
                                                                 : sizeof(Merge16<NW>);
}
constexpr float kRescale16 = 8.0f;

#ifndef BD3_DEC16_OCC
#define BD3_DEC16_OCC 4
#endif

template <int NW>
__global__ __launch_bounds__(NW * 64, BD3_DEC16_OCC) void decode16_partial(DecodeArgs a) {
  constexpr int kNT = NW * 64;
  __shared__ __attribute__((aligned(16))) char smem[smem16_bytes<NW>()];
  const int tid = wi_x();
  const int lane = tid & 63;
  const int wave = wave_uniform(tid >> 6);
  const int l16 = lane & 15;
  const int hq = lane >> 4;  // 16-lane group
  __bf16* ks = reinterpret_cast<__bf16*>(smem) + wave * 2 * kTile16;
  __bf16* vs = ks + kTile16;

  const int grp = wg_x();
  const int bh = wg_z();
  const int b = bh / a.heads, h = bh - b * a.heads;
  const uint16_t* qp = a.q + b * a.sq.b + h * a.sq.h;
  const uint16_t* kp = a.k + b * a.sk.b + h * a.sk.h;
  const uint16_t* vp = a.v + b * a.sv.b + h * a.sv.h;

  const int qrow = imin(l16, a.q_len - 1);
  bf16x8 qreg[2];
#pragma unroll
  for (int c = 0; c < 2; ++c)
    qreg[c] = __builtin_bit_cast(bf16x8, ld16(qp + (int64_t)qrow * a.sq.s + 32 * c + 8 * hq));
  // Row l16 sees keys [0, khi); rows past q_len are computed and dropped.
  const int pos = a.kv_len - a.q_len + l16;
  const int khi = l16 < a.q_len ? imin((pos / a.bs + 1) * a.bs, a.kv_len) : a.kv_len;

  const int key_end = wave_uniform(decode_key_end(0, kQ16, a.q_len, a.kv_len, a.bs));
  // keys below kfull are seen by every row (row 0 has the smallest position)
  const int kfull = wave_uniform(imin(((a.kv_len - a.q_len) / a.bs + 1) * a.bs, a.kv_len));
  const int tr_row = l16 >> 2;
  const int tr_col = 4 * (lane & 3);

  // lane + 64j -> key row c0 + lane/8 + 8j, 16-byte part lane%8
  u32x4 kr[kLoads16], vr[kLoads16];
  auto load = [&](int c0) {
#pragma unroll
    for (int j = 0; j < kLoads16; ++j) {
      const int key = imin(c0 + (lane >> 3) + 8 * j, a.kv_len - 1);
      kr[j] = ld16_stream(kp + (int64_t)key * a.sk.s + 8 * (lane & 7));
    }
#pragma unroll
    for (int j = 0; j < kLoads16; ++j) {
      const int key = imin(c0 + (lane >> 3) + 8 * j, a.kv_len - 1);
      vr[j] = ld16_stream(vp + (int64_t)key * a.sv.s + 8 * (lane & 7));
    }
  };

  // One 32-key chunk starting at c0 (keys from hi on are the next split's or
  // invisible), already in the wave's LDS tiles, into the online-softmax
  // state (m, lsum, o): lsum is the lane's share of the row sum (its 8 keys
  // per chunk), o is O^T unnormalised ([16-d block]: lane (row l16, hq) holds
  // d 16db + 4hq + r).
  auto chunk = [&](int c0, int hi, float& m, float& lsum, f32x4 (&o)[4]) {
    f32x4 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const __bf16* kt = &ks[(16 * kb + l16) * kStride + 8 * hq];
      s[kb] = mfma16(*reinterpret_cast<const bf16x8*>(kt), qreg[0], f32x4{});
      s[kb] = mfma16(*reinterpret_cast<const bf16x8*>(kt + 32), qreg[1], s[kb]);
    }
    if (c0 + kChunk16 > kfull || c0 + kChunk16 > hi) {  // partial chunk (uniform)
      const int lim = imin(khi, hi);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          s[kb][r] = (c0 + 16 * kb + 4 * hq + r < lim) ? s[kb][r] : -INFINITY;
    }
    float mx = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                     fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3])));
    mx = fmaxf(mx, shfl_xor(mx, 16));
    mx = max_xor32(mx);
    const float mt = mx * a.scale_log2;
    if (__ballot(mt > m + kRescale16) != 0) {
      const float mn = fmaxf(m, mt);
      const float alpha = (mn == -INFINITY) ? 1.f : fast_exp2(m - mn);
      m = mn;
      lsum *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db) o[db] *= alpha;
    }
    const float mu = (m == -INFINITY) ? 0.f : m;
    float p[2][4];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p[kb][r] = fast_exp2(fmaf(s[kb][r], a.scale_log2, -mu));
        lsum += p[kb][r];
      }
    const bf16x8 pop = to_bf16x8(p[0][0], p[0][1], p[0][2], p[0][3], p[1][0], p[1][1], p[1][2], p[1][3]);
    const int row = 4 * hq + tr_row;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const bf16x8 va = cat8(lds_read_tr(&vs[row * kStride + 16 * db + tr_col]),
                             lds_read_tr(&vs[(row + 16) * kStride + 16 * db + tr_col]));
      o[db] = mfma16(va, pop, o[db]);
    }
  };
  // The chunk loaded last (registers) to the wave's LDS tiles.
  auto stage = [&]() {
#pragma unroll
    for (int j = 0; j < kLoads16; ++j) {
      const int off = ((lane >> 3) + 8 * j) * kStride + 8 * (lane & 7);
      *reinterpret_cast<u32x4*>(&ks[off]) = kr[j];
      *reinterpret_cast<u32x4*>(&vs[off]) = vr[j];
    }
  };
  // Chunk i of a split's walk is chunk (i + r0) mod n_chunks of the split
  // (r0 = 7 bh mod n_chunks, the same for every wave). Without that rotation
  // every workgroup reads the same offset of its head's K/V at the same
  // time, and the head stride (kv_len x 128 bytes) piles those reads onto
  // few HBM channels; starting head bh at chunk 7 bh spreads them (measured
  // 71 -> 66 us at 32 x 12 heads, kv_len 4112, one split).
  auto split_lo = [&](int sp) { return wave_uniform(sp * a.split_len); };
  auto split_hi = [&](int sp) { return wave_uniform(imin(sp * a.split_len + a.split_len, key_end)); };
  auto n_chunks_of = [&](int sp) {
    const int lo = split_lo(sp), hi = split_hi(sp);
    return hi > lo ? (hi - lo + kChunk16 - 1) / kChunk16 : 0;
  };
  int crot = bh * 7;  // start rotation of the chunks inside a split (mod its chunk count)
  auto chunk_c0 = [&](int sp, int nc, int i) {
    const int c = i + (nc > 0 ? crot % nc : 0);
    return split_lo(sp) + (c >= nc ? c - nc : c) * kChunk16;
  };

  // The wave's state for the workgroup merge: weights 2^(m - max m), sums l,
  // unnormalised O (lane shares of l, summed below).
  f32x4 o[4] = {};
  float m = -INFINITY, lsum = 0.f;
  const int s0 = wave_uniform(grp * a.splits_per_group);
  const int s1 = wave_uniform(imin(s0 + a.splits_per_group, a.n_splits));
  if (a.splits_per_group == 1) {
    // One split per workgroup: the waves take its chunks in turn; each
    // wave's next chunk streams in while the current one is computed.
    const int hi = split_hi(s0);
    const int nc = n_chunks_of(s0);
    if (wave < nc) load(chunk_c0(s0, nc, wave));
    for (int ch = wave; ch < nc; ch += NW) {
      stage();
      if (ch + NW < nc) load(chunk_c0(s0, nc, ch + NW));
      chunk(chunk_c0(s0, nc, ch), hi, m, lsum, o);
    }
  } else {
    // Several splits per workgroup, computed one after another; the waves
    // take the chunks in turn (the one-split read pattern). A
    // wave's share of a split gives a normalised partial and its log2-LSE
    // (the reference's per-split result, kernels/SplitKVDecodeAttention.py:
    // 81-87, over the wave's keys of the split), merged into the wave's
    // running state with the reference's LSE weights (:109-127); the
    // workgroup merge below combines the waves the same way. The lane shares
    // of l stay unreduced: m and O are per row, the weights apply to every
    // share. The next chunk's loads (at a split's end, the wave's first
    // chunk of the next split) stream in while the current chunk is computed.
    // The workgroup's chunks, split after split, are dealt to the waves in
    // turn (chunk g of the sequence to wave g mod NW), so every wave gets the
    // same count to within one whatever the chunks per split. The head
    // starts where the one-split order starts it, chunk 7 bh of its chunks
    // (mod their count): the splits are visited from the one holding that
    // chunk on (j-th visited: s0 + (j + rot) mod cnt) and each split's chunks
    // from the same offset on, so heads read different parts of their caches
    // at any moment (the merge is order-independent up to rounding).
    const int cnt = s1 - s0;
    const int ncf = wave_uniform(imax(a.split_len / kChunk16, 1));  // chunks of a full split
    const int start = wave_uniform((bh * 7) % (cnt * ncf));
    const int rot = wave_uniform(start / ncf);
    crot = start - rot * ncf;
    auto act = [&](int j) { return s0 + (j + rot >= cnt ? j + rot - cnt : j + rot); };
    int vs = 0, nc = n_chunks_of(act(0)), i = wave;
    while (vs < cnt && i >= nc) {
      i -= nc;
      ++vs;
      nc = vs < cnt ? n_chunks_of(act(vs)) : 0;
    }
    if (vs < cnt) load(chunk_c0(act(vs), nc, i));
    float ms = -INFINITY, ls = 0.f;
    f32x4 os[4] = {};
    while (vs < cnt) {
      stage();
      int vs_n = vs, nc_n = nc, i_n = i + NW;
      while (vs_n < cnt && i_n >= nc_n) {
        i_n -= nc_n;
        ++vs_n;
        nc_n = vs_n < cnt ? n_chunks_of(act(vs_n)) : 0;
      }
      if (vs_n < cnt) load(chunk_c0(act(vs_n), nc_n, i_n));
      const int sp = act(vs);
      chunk(chunk_c0(sp, nc, i), split_hi(sp), ms, ls, os);
      if (vs_n != vs) {
        // the wave's share of split sp is done: merge its normalised partial
        float lrow = ls + shfl_xor(ls, 16);
        lrow = sum_xor32(lrow);
        if (lrow > 0.f) {
          const float lse = ms + fast_log2(lrow);  // log2-LSE of the share
          const float mn = fmaxf(m, lse);
          const float w_old = m == -INFINITY ? 0.f : fast_exp2(m - mn);
          const float w_new = fast_exp2(lse - mn) / lrow;  // weight of the normalised partial
          m = mn;
          // running state: each of the row's 4 lane shares holds a quarter of l
          lsum = lsum * w_old + 0.25f * fast_exp2(lse - mn);
#pragma unroll
          for (int db = 0; db < 4; ++db) o[db] = o[db] * w_old + os[db] * w_new;
        }
        ms = -INFINITY;
        ls = 0.f;
#pragma unroll
        for (int db = 0; db < 4; ++db) os[db] = f32x4{};
      }
      vs = vs_n;
      nc = nc_n;
      i = i_n;
    }
  }

  // Merge the waves' states.
  lsum += shfl_xor(lsum, 16);
  lsum = sum_xor32(lsum);
  __syncthreads();  // the K/V tiles are reused below
  Merge16<NW>* ml = reinterpret_cast<Merge16<NW>*>(smem);
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int r = 0; r < 4; ++r) ml->o[wave][16 * db + 4 * hq + r][l16] = o[db][r];
  if (hq == 0) {
    ml->m[wave][l16] = m;
    ml->l[wave][l16] = lsum;
  }
  __syncthreads();

  // kNT threads x kOut outputs = 16 rows x 64 d.
  constexpr int kOut = kQ16 * kHeadDim / kNT;
  constexpr int kTPR = kHeadDim / kOut;  // threads per row
  const int row = tid / kTPR, d0 = kOut * (tid % kTPR);
  float mm = -INFINITY;
#pragma unroll
  for (int w = 0; w < NW; ++w) mm = fmaxf(mm, ml->m[w][row]);
  const float mu = (mm == -INFINITY) ? 0.f : mm;
  float lt = 0.f;
  float ot[kOut] = {};
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const float wgt = fast_exp2(ml->m[w][row] - mu);
    lt += wgt * ml->l[w][row];
#pragma unroll
    for (int j = 0; j < kOut; ++j) ot[j] += wgt * ml->o[w][d0 + j][row];
  }
  if (a.groups == 1) {
    if (row < a.q_len) {
      const float inv = 1.f / lt;
      uint16_t* dst = a.o + b * a.so.b + h * a.so.h + (int64_t)row * a.so.s + d0;
      if constexpr (kOut == 2) {
        const bf16x4 y = to_bf16x4(ot[0] * inv, ot[1] * inv, 0.f, 0.f);
        *reinterpret_cast<bf16x2*>(dst) = bf16x2{y[0], y[1]};
      } else {
#pragma unroll
        for (int j = 0; j < kOut; j += 4)
          *reinterpret_cast<bf16x4*>(dst + j) =
              to_bf16x4(ot[j] * inv, ot[j + 1] * inv, ot[j + 2] * inv, ot[j + 3] * inv);
      }
    }
  } else {
    const int64_t slot = (int64_t)bh * a.q_tiles * a.groups + grp;  // q_tiles == 1
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    float* dst = &a.part_o[(slot * kQT + row) * kHeadDim + d0];
#pragma unroll
    for (int j = 0; j < kOut; ++j) dst[j] = ot[j] * inv;
    if (tid % kTPR == 0) a.part_lse[slot * kQT + row] = lt > 0.f ? mm + fast_log2(lt) : -INFINITY;
  }
}

// Split merge: thread -> (row, 4 consecutive d); rows in passes of 16. For
// NS > 0 the call has at most NS splits and all loads of a row are issued
// before the first use (one memory round trip); NS == 0 takes any count.
template <int NS>
__global__ __launch_bounds__(kThreads) void decode_combine(DecodeArgs a) {
  const int qt = wg_x();
  const int bh = wg_y();
  const int b = bh / a.heads, h = bh - b * a.heads;
  const int i0 = qt * kQT;
  uint16_t* op = a.o + b * a.so.b + h * a.so.h;
  const int64_t slot0 = ((int64_t)bh * a.q_tiles + qt) * a.groups;
  const int d0 = 4 * (wi_x() & 15);
#pragma unroll
  for (int pass = 0; pass < kQT / 16; ++pass) {
    const int row = pass * 16 + (wi_x() >> 4);
    if (i0 + row >= a.q_len) continue;
    const float* lp = a.part_lse + slot0 * kQT + row;                  // split s: lp[s * kQT]
    const float* pp = a.part_o + (slot0 * kQT + row) * kHeadDim + d0;  // split s: pp[s * kQT * kHeadDim]
    float mm = -INFINITY, wt = 0.f;
    f32x4 acc = {};
    if constexpr (NS > 0) {
      const int ns = a.groups;  // <= NS
      float l[NS];
      f32x4 po[NS];
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        if (s < ns) {
          l[s] = lp[s * kQT];
          po[s] = *reinterpret_cast<const f32x4*>(pp + s * kQT * kHeadDim);
        } else {
          l[s] = -INFINITY;
          po[s] = f32x4{};
        }
      }
#pragma unroll
      for (int s = 0; s < NS; ++s) mm = fmaxf(mm, l[s]);
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const float w = s < ns ? fast_exp2(l[s] - mm) : 0.f;  // empty split -> 0
        wt += w;
        acc += w * po[s];
      }
    } else {
      // Any count, 8 splits per memory round trip (all loads of a group are
      // issued before the first use); the same weights, summed in split
      // order.
      constexpr int kG = 8;
      const int ns = a.groups;
      for (int s0 = 0; s0 < ns; s0 += kG) {
        float l[kG];
#pragma unroll
        for (int k = 0; k < kG; ++k) l[k] = s0 + k < ns ? lp[(s0 + k) * kQT] : -INFINITY;
#pragma unroll
        for (int k = 0; k < kG; ++k) mm = fmaxf(mm, l[k]);
      }
      for (int s0 = 0; s0 < ns; s0 += kG) {
        float l[kG];
        f32x4 po[kG];
#pragma unroll
        for (int k = 0; k < kG; ++k) {
          if (s0 + k < ns) {
            l[k] = lp[(s0 + k) * kQT];
            po[k] = *reinterpret_cast<const f32x4*>(pp + (s0 + k) * kQT * kHeadDim);
          }
        }
#pragma unroll
        for (int k = 0; k < kG; ++k) {
          if (s0 + k < ns) {
            const float w = fast_exp2(l[k] - mm);
            wt += w;
            acc += w * po[k];
          }
        }
      }
    }
    const float inv = 1.f / wt;
    *reinterpret_cast<bf16x4*>(op + (int64_t)(i0 + row) * a.so.s + d0) =
        to_bf16x4(acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv);
  }
}

__global__ void mask_dump_kernel(uint8_t* out, int mode, int rows, int cols, int kv_len,
                                 int bs) {
  const int64_t e = (int64_t)wg_x() * 256 + wi_x();
  if (e >= (int64_t)rows * cols) return;
  const int i = (int)(e / cols), j = (int)(e - (int64_t)i * cols);
  bool vis;
  if (mode == 0) {
    vis = train_visible(i, j, rows / 2, bs);
  } else {
    vis = decode_visible(i, j, rows, kv_len, bs);
  }
  out[e] = vis ? 1 : 0;
}

}  // namespace

hipError_t launch_decode(const DecodeArgs& a, int /*qt*/, hipStream_t stream) {
  dim3 grid(a.groups, a.q_tiles, a.bh);
  if (a.q_len <= kQ16)
    hipLaunchKernelGGL(decode16_partial<kNW>, grid, dim3(kThreads), 0, stream, a);
  else if ((int64_t)a.bh * a.q_tiles * a.groups < 256 && a.split_len >= 512)
    // Fewer workgroups than CUs, each with at least 16 chunks: 8 waves share
    // them (measured at 8 x 12 heads, q_len 32, one split: 2048 keys 20.9 ->
    // 17.8 us, 1024 keys 13.4 -> 12.0; batch 1 over 3584 keys 30.1 -> 22.3;
    // with 128 keys per split 4 waves stay faster, 7.1 vs 7.6 us).
    hipLaunchKernelGGL(decode_partial<8>, grid, dim3(8 * 64), 0, stream, a);
  else
    hipLaunchKernelGGL(decode_partial<kNW>, grid, dim3(kThreads), 0, stream, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.groups == 1) return e;
  const dim3 cgrid(a.q_tiles, a.bh);
  if (a.groups == 2)
    hipLaunchKernelGGL(decode_combine<2>, cgrid, dim3(kThreads), 0, stream, a);
  else if (a.groups == 3)
    hipLaunchKernelGGL(decode_combine<3>, cgrid, dim3(kThreads), 0, stream, a);
  else if (a.groups == 4)
    hipLaunchKernelGGL(decode_combine<4>, cgrid, dim3(kThreads), 0, stream, a);
  else if (a.groups <= 16)
    hipLaunchKernelGGL(decode_combine<16>, cgrid, dim3(kThreads), 0, stream, a);
  else if (a.groups <= 32)
    hipLaunchKernelGGL(decode_combine<32>, cgrid, dim3(kThreads), 0, stream, a);
  else
    hipLaunchKernelGGL(decode_combine<0>, cgrid, dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_mask_dump(uint8_t* out, int mode, int rows, int kv_len, int bs,
                            hipStream_t stream) {
  const int r = mode == 0 ? 2 * rows : rows;
  const int c = mode == 0 ? 2 * rows : kv_len;
  const int64_t total = (int64_t)r * c;
  hipLaunchKernelGGL(mask_dump_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream,
                     out, mode, r, c, kv_len, bs);
  return hipGetLastError();
}

}  // namespace bd3
