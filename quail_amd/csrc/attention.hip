// Paged varlen causal GQA attention over the KV arena, with the o_proj input
// quantization fused into the epilogue. Replaces the FlashAttention varlen
// call of quail/backends/quail/executor/attention.py:1280-1306 (reached from
// attention_unified :1558-1563 through _paged :1368-1393) followed by the
// per-token group quant of :1274-1275.
//
// Semantics (FA varlen with block_table and seqused_k):
//   sequence s owns query rows [cu_q[s], cu_q[s+1]) and reads keys [0, used[s])
//   through table[s] (page ids, `page` tokens per page). With causal masking
//   the alignment is bottom-right: query i (0-based in s) of a sequence with
//   q_len rows sees keys < used[s] - q_len + i + 1. Scale 1/sqrt(D) by default.
//   GQA: query head h reads KV head h / (HQ / HK).
//   Pools: k_pool, v_pool are (pages * page, HK, D) bf16.
//
// Output: bf16 (n, HQ*D), or with D == 128 the e4m3 o_proj input (n, HQ*D)
// plus fp32 scales at scales[h * s_ld + row] (one 128-group = one head),
// computed from the bf16-rounded attention output exactly as the reference's
// separate quant kernel would see it.
//
// Kernel layout (CDNA4). A workgroup is QSUB 32-row query tiles of one
// sequence x HPB query heads sharing one KV head: one wave per (tile, head),
// so every K/V tile staged in LDS serves HPB * QSUB * 32 query rows. KV is
// consumed in 64-key tiles, software pipelined: each step computes S of the
// next tile beside the softmax and PV of the current one, while K and V rows
// of later tiles travel HBM -> LDS directly (global_load_lds) into double
// buffers; one barrier per step. The sequence's page-table row is staged in LDS once.
//
// Each wave forms S^T = K Q^T with v_mfma_f32_32x32x16_bf16 so that a lane
// owns one query column; the online softmax is then lane-local (plus one
// cross-half shuffle), P^T feeds the PV MFMA directly as its B operand, and
// O^T keeps one query per lane, so rescaling needs no shuffles. The V^T
// operand of the PV MFMA comes straight from the row-major V tile through
// gfx950's transposing LDS read (ds_read_b64_tr_b16). The PV product runs in
// the V pool's 16-bit type: bf16, as the reference's FlashAttention does with
// the bf16 pools of its arena, or fp16 for an arena that stores V in fp16
// (P then keeps 11 significant bits instead of 8); the row sums take the
// unrounded fp32 P.
#include <algorithm>
#include <type_traits>
#include <vector>

#include "qx_common.h"
#include "qx_status.h"

namespace qx {
namespace {

typedef __attribute__((address_space(3))) void lds_void;

constexpr int kBK = 64;          // keys per KV tile
constexpr int kPage = 16;        // tokens per arena page
// page-table entries staged in LDS per sequence: 40,960 keys at 16-row
// pages, Qwen3's whole context (two workgroups' 74.5 KiB still fit a CU)
constexpr int kMaxPages = 2560;
// a row's reference max moves when a tile raises its max by more than this
// many powers of two (probabilities then stay below 2^8)
constexpr float kLazyLog2 = 8.0f;

typedef short v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s lds_v4s;

// 16-B chunk swizzle of a K row (2*D bytes): the 16 rows of one ds_read_b128
// phase map to 16 distinct 16-B bank groups of the 64-bank LDS
template <int D>
__device__ __forceinline__ int kswz(int key) { return D == 128 ? (key & 15) : ((key >> 1) & 7); }

// 16-B chunk swizzle of a V row: one transposing read covers 4 consecutive
// keys x 4 chunks per 32-lane phase, which land in 16 distinct bank groups
template <int D>
__device__ __forceinline__ int vswz(int key) { return D == 128 ? ((key & 3) << 2) : (((key >> 1) & 1) << 2); }

// QN != 0: q holds the raw (pre-norm) q columns of the qkv projection, and
// the kernel applies each row's qk-norm and RoPE as it loads it: position
// pos[row], the cos/sin cache cs ((max_pos, 128) [cos | sin], bf16 for
// QN = 1, fp32 for QN = 2), the q-norm weight qw and eps.
struct QNormArgs {
  const int64_t* pos;
  const void* cs;       // (positions, 128) cos | sin; bf16 (QN 1) or fp32 (QN 2)
  const uint16_t* qw;  // the q-norm weight (128), bf16
  float eps;
};

// What q-norm on load reads for one lane: the q-norm weight of its 64
// columns (c*16 + half*8 + k, c, k < 8), then, once the row's position is
// in, the row's cos / sin of its first-half columns (bf16 for QN = 1, fp32
// for QN = 2), raw as loaded.
template <int QN>
struct QNormIn {
  static constexpr int kCs = QN == 2 ? 16 : 8;
  uint4 wq[8];
  uint4 cs[kCs];
};

template <int QN>
__device__ __forceinline__ void q_norm_load_weights(QNormIn<QN>& in, const QNormArgs& qn,
                                                    int half) {
#pragma unroll
  for (int c = 0; c < 8; ++c)
    in.wq[c] = *reinterpret_cast<const uint4*>(qn.qw + c * 16 + half * 8);
}

template <int QN>
__device__ __forceinline__ void q_norm_load_row(QNormIn<QN>& in, const QNormArgs& qn, int64_t p,
                                                int half) {
  if constexpr (QN == 1) {
    const uint16_t* row_cs = reinterpret_cast<const uint16_t*>(qn.cs) + p * 128;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      in.cs[2 * c] = *reinterpret_cast<const uint4*>(row_cs + c * 16 + half * 8);
      in.cs[2 * c + 1] = *reinterpret_cast<const uint4*>(row_cs + 64 + c * 16 + half * 8);
    }
  } else {
    const float* row_cs = reinterpret_cast<const float*>(qn.cs) + p * 128;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        in.cs[4 * c + 2 * e] = *reinterpret_cast<const uint4*>(row_cs + c * 16 + half * 8 + e * 4);
        in.cs[4 * c + 2 * e + 1] =
            *reinterpret_cast<const uint4*>(row_cs + 64 + c * 16 + half * 8 + e * 4);
      }
  }
}

// The lane's 64 q columns of one head through qk-norm and RoPE with the
// qk-norm-rope pass's arithmetic and summation tree. The pass sums a head's
// 16 column groups j (columns 4j.. and 64 + 4j..) with a butterfly over j
// (xor 8, 4, 2, 1); group j = 4c + 2 half + e (c < 4) is this lane's
// columns c*16 + half*8 + 4e.., so the xor-8 and xor-4 levels pair the
// lane's own groups (c ^ 2, c ^ 1), xor 2 pairs it with lane ^ 32 and xor 1
// its own e ^ 1: the same sums of the same terms, and each addition
// commutes, so the rows come out bit for bit as the pass writes them.
template <int QN>
__device__ __forceinline__ void q_norm_rope_apply(v8s (&qf)[8], const QNormIn<QN>& in,
                                                  float eps) {
  float cosv[4][2][4], sinv[4][2][4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    if constexpr (QN == 1) {
      const uint4 cw = in.cs[2 * c], sw = in.cs[2 * c + 1];
      bf16x4_to_f32(make_uint2(cw.x, cw.y), cosv[c][0]);
      bf16x4_to_f32(make_uint2(cw.z, cw.w), cosv[c][1]);
      bf16x4_to_f32(make_uint2(sw.x, sw.y), sinv[c][0]);
      bf16x4_to_f32(make_uint2(sw.z, sw.w), sinv[c][1]);
    } else {
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const uint4 cv = in.cs[4 * c + 2 * e], sv = in.cs[4 * c + 2 * e + 1];
        cosv[c][e][0] = __uint_as_float(cv.x); cosv[c][e][1] = __uint_as_float(cv.y);
        cosv[c][e][2] = __uint_as_float(cv.z); cosv[c][e][3] = __uint_as_float(cv.w);
        sinv[c][e][0] = __uint_as_float(sv.x); sinv[c][e][1] = __uint_as_float(sv.y);
        sinv[c][e][2] = __uint_as_float(sv.z); sinv[c][e][3] = __uint_as_float(sv.w);
      }
    }
  }
  auto group = [&](const v8s& x, int e, float (&out)[4]) {
    const uint4 w = __builtin_bit_cast(uint4, x);
    bf16x4_to_f32(e ? make_uint2(w.z, w.w) : make_uint2(w.x, w.y), out);
  };
  float s[4][2];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      float a[4], b[4];
      group(qf[c], e, a);
      group(qf[c + 4], e, b);
      s[c][e] = norm_part4(a, b);
    }
  float w[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) w[e] = sum_halves((s[0][e] + s[2][e]) + (s[1][e] + s[3][e]));
  const float rstd = norm_rstd<128>(w[0] + w[1], eps);
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    uint4 lo = __builtin_bit_cast(uint4, qf[c]), hi = __builtin_bit_cast(uint4, qf[c + 4]);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      float a[4], b[4], wa[4], wb[4], oa[4], ob[4];
      group(qf[c], e, a);
      group(qf[c + 4], e, b);
      group(__builtin_bit_cast(v8s, in.wq[c]), e, wa);
      group(__builtin_bit_cast(v8s, in.wq[c + 4]), e, wb);
      norm_rope4(a, b, wa, wb, cosv[c][e], sinv[c][e], rstd, oa, ob);
      const uint32_t o0 = pack2_bf16(oa[0], oa[1]), o1 = pack2_bf16(oa[2], oa[3]);
      const uint32_t p0 = pack2_bf16(ob[0], ob[1]), p1 = pack2_bf16(ob[2], ob[3]);
      if (e) {
        lo.z = o0; lo.w = o1; hi.z = p0; hi.w = p1;
      } else {
        lo.x = o0; lo.y = o1; hi.x = p0; hi.y = p1;
      }
    }
    qf[c] = __builtin_bit_cast(v8s, lo);
    qf[c + 4] = __builtin_bit_cast(v8s, hi);
  }
}

// CONTIG: keys are contiguous rows, key j of sequence s at row cu_k[s] + j
// (no block table). q_index (optional): query row i reads Q row q_index[i].
// lse (optional): lse[h * lse_ld + i] = ln(sum_j exp(scale * s_ij)) of row i.
// VBF: the V pool holds bf16 and the PV product runs in bf16 (P rounded to
// bf16); otherwise V holds fp16 and P is rounded to fp16 (11 significant
// bits against bf16's 8: the closer result, for an arena of this engine's
// own that stores V in fp16).
// Registers for two waves per SIMD: one 8-wave workgroup per CU, or two of
// 4 waves.
template <int D, int HPB, int QSUB, bool QUANT, bool CONTIG, bool VBF, int QN = 0>
__global__ __launch_bounds__(HPB * QSUB * 64, 8 / (HPB * QSUB)) void paged_attention_kernel(
    const uint16_t* __restrict__ q, int64_t q_ld, const int64_t* __restrict__ q_index,
    const uint16_t* __restrict__ kp, const uint16_t* __restrict__ vp,
    const int* __restrict__ cu_q, const int* __restrict__ used, const int* __restrict__ table,
    int64_t table_ld, const int* __restrict__ cu_k, int max_used, int HQ, int HK,
    float scale_log2, int causal, uint16_t* __restrict__ out16, uint8_t* __restrict__ out8,
    int64_t o_ld, float* __restrict__ scales, int64_t s_ld, float* __restrict__ lse,
    int64_t lse_ld, const int* __restrict__ work, int zgroups, int seqs, QNormArgs qn) {
  static_assert(QN == 0 || (D == 128 && QUANT && !CONTIG), "q-norm on load: the paged D=128 call");
  constexpr int NW = HPB * QSUB;
  constexpr int NT = NW * 64;
  constexpr int BQ = 32 * QSUB;  // query rows per workgroup
  constexpr int ND16 = D / 16;   // MFMA k-steps over the head dim
  constexpr int NDS = D / 32;    // 32-row d tiles of O^T
  constexpr int KCH = D / 8;     // 16-byte chunks per K or V row
  constexpr int ROW = D * 2;     // bytes per K or V row
  constexpr int T_BYTES = kBK * ROW;
  constexpr int KEYS_PER_SLAB = 1024 / ROW;         // keys per direct-load instruction
  constexpr int SLABS = kBK / KEYS_PER_SLAB / NW;   // per wave per tile, for K and for V
  static_assert(SLABS >= 1 && SLABS * KEYS_PER_SLAB * NW == kBK, "slabs");
  // separate objects per buffer, so the compiler can see that the direct
  // loads into one buffer never alias the reads of the other
  __shared__ __attribute__((aligned(1024))) uint8_t kv_lds[2][2][T_BYTES];  // [buffer][K, V]
  auto k_buf = [&](int b) -> uint8_t* { return &kv_lds[b][0][0]; };
  auto v_buf = [&](int b) -> uint8_t* { return &kv_lds[b][1][0]; };
  __shared__ int pages_lds[kMaxPages + 64];  // + one wave's DMA past the last page

  // the workgroup's (sequence, query tile, head group): from the work list
  // (one item per real query tile, heaviest first, head groups innermost),
  // or from the full grid (late query tiles first)
  int s, qt, zg;
  if (work) {
    const int item = blockIdx.x / zgroups;
    zg = blockIdx.x % zgroups;
    s = work[2 * item];
    qt = work[2 * item + 1];
  } else {
    s = blockIdx.y;
    qt = gridDim.x - 1 - blockIdx.x;
    zg = blockIdx.z;
  }
  // the sequence's bounds in one round of loads (s clamped into range, so
  // every load is in bounds), then the exits: each dependent load is a
  // memory round trip before the first KV tile
  const int sc = min(max(s, 0), seqs - 1);
  const int q0 = cu_q[sc];
  const int q_len = cu_q[sc + 1] - q0;
  const int used_raw = used[sc];
  const int kv_first = CONTIG ? cu_k[sc] : 0;
  if (s < 0 || s >= seqs || qt < 0) return;  // not an item of this call
  if (qt * BQ >= q_len) return;               // uniform over the workgroup
  const int G = HQ / HK;
  const int groups_per_kv = G / HPB;
  const int kvh = zg / groups_per_kv;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int head = kvh * G + (zg % groups_per_kv) * HPB + (wave % HPB);
  const int qsub = wave / HPB;
  const int half = lane >> 5;
  const int col = lane & 31;

  const int used_s = min(used_raw, max_used);
  const int off = causal ? used_s - q_len : 0;
  const int r = qt * BQ + qsub * 32 + col;  // this lane's query row within the sequence
  const bool r_ok = r < q_len;
  const int block_last = min(qt * BQ + BQ, q_len) - 1;
  const int kv_end = max(0, causal ? min(used_s, off + block_last + 1) : used_s);
  // keys this wave can see at all (its last valid row)
  const int wave_last = min(qt * BQ + qsub * 32 + 31, q_len - 1);
  const int wave_end = causal ? min(used_s, off + wave_last + 1) : used_s;
  const int ntiles = (kv_end + kBK - 1) / kBK;

  // this lane's Q row (through q_index, which only the tree path's reads of
  // resident pages pass, before the table load so that its wait does not
  // also wait for that)
  int64_t qr;
  {
    const int rr = r_ok ? r : q_len - 1;
    const int64_t* qi = QUANT ? nullptr : q_index;
    qr = qi ? qi[q0 + rr] : (int64_t)(q0 + rr);
  }
  const uint16_t* qrow = q + qr * q_ld + head * D;

  // stage the page-table row straight into LDS (no VGPR round trip), in
  // flight together with the Q loads below: 64 entries per wave and pass,
  // lanes past the row's last page re-read it (their LDS slots, inside the
  // padding, are never read)
  const int kv0 = kv_first;
  if (!CONTIG) {
    const int* trow = table + (int64_t)s * table_ld;
    const int npages = (kv_end + kPage - 1) / kPage;
    for (int b = wave * 64; b < npages; b += NT)
      lds_dma4(trow + min(b + lane, npages - 1), (const uint8_t*)&pages_lds[b]);
  }

  // Q^T fragments (B operand): lane holds query `col`, d = c*16 + half*8 .. +8
  v8s qf[ND16];
  // q-norm on load: the row's position and the weights go out with Q; the
  // row's cos / sin (which need the position) after it, with the first K
  // and V tiles, so that one memory round trip covers both
  QNormIn<QN == 0 ? 1 : QN> qin;
  int64_t q_pos = 0;
  {
    if constexpr (QN != 0) q_pos = qn.pos[qr];
#pragma unroll
    for (int c = 0; c < ND16; ++c) qf[c] = *reinterpret_cast<const v8s*>(qrow + c * 16 + half * 8);
    if constexpr (QN != 0) q_norm_load_weights(qin, qn, half);
    // consume the Q fragments here, before any KV load is issued: the
    // compiler's own waits for them would otherwise land inside the tile
    // loop, behind the KV loads it does not track, and drain those too
#pragma unroll
    for (int c = 0; c < ND16; ++c) asm volatile("" ::"v"(qf[c]));
  }
  const int64_t kv_row = (int64_t)HK * D;  // elements per pool row
  const uint16_t* kbase = kp + kvh * D;
  const uint16_t* vbase = vp + kvh * D;
  __builtin_amdgcn_s_waitcnt(0);
  if constexpr (QN != 0) q_norm_load_row(qin, qn, q_pos, half);
  lds_barrier();  // pages_lds visible

  // K (or V) rows of tile t straight into LDS: lane i of a slab writes bytes
  // [16i, 16i+16): key i / KCH of the slab, physical chunk i % KCH, which
  // holds logical chunk (i % KCH) ^ swizzle(key); keys past the last (in
  // the last tile) re-read the last key (in bounds, never used)
  // A wave's KPW keys of a tile lie in one page (KPW divides the page and
  // the wave's first key is a multiple of KPW): for a tile wholly below
  // kv_end each lane's address is the page's first row (wave-uniform) plus
  // a byte offset that is the same for every tile
  constexpr int KPW = kBK / NW;
  static_assert(KPW * NW == kBK && kPage % KPW == 0 && SLABS * KEYS_PER_SLAB == KPW, "page slabs");
  uint32_t koff[SLABS], voff[SLABS];
#pragma unroll
  for (int j = 0; j < SLABS; ++j) {
    const int key = (wave * SLABS + j) * KEYS_PER_SLAB + lane / KCH;  // key within the tile
    const uint32_t in_page = (uint32_t)((wave * KPW) % kPage + j * KEYS_PER_SLAB + lane / KCH);
    const int p = lane % KCH;
    koff[j] = in_page * (uint32_t)(kv_row * 2) + (uint32_t)((p ^ kswz<D>(key)) * 16);
    voff[j] = in_page * (uint32_t)(kv_row * 2) + (uint32_t)((p ^ vswz<D>(key)) * 16);
  }
  auto issue = [&](int t, int buf, bool v) {
    if (t * kBK + kBK <= kv_end) {
      const int page_slot = t * (kBK / kPage) + (wave * KPW) / kPage;
      const int64_t row0 =
          CONTIG ? (int64_t)kv0 + t * kBK + ((wave * KPW) / kPage) * kPage
                 : (int64_t)__builtin_amdgcn_readfirstlane(pages_lds[page_slot]) * kPage;
      const uint8_t* src = reinterpret_cast<const uint8_t*>((v ? vbase : kbase) + row0 * kv_row);
#pragma unroll
      for (int j = 0; j < SLABS; ++j) {
        const int slab = wave * SLABS + j;
        lds_dma16(src + (v ? voff[j] : koff[j]), (v ? v_buf(buf) : k_buf(buf)) + slab * 1024);
      }
      return;
    }
    // the item's last tile: the same page-based addresses for the keys below
    // kv_end; the rest re-read the last key's row (its page read once too)
    const int kv_last = kv_end - 1;
    const int wave_key0 = t * kBK + wave * KPW;
    const int page_key0 = (min(wave_key0, kv_last) / kPage) * kPage;
    int64_t row0, row_last;
    if (CONTIG) {
      row0 = (int64_t)kv0 + page_key0;
      row_last = (int64_t)kv0 + kv_last;
    } else {
      row0 = (int64_t)__builtin_amdgcn_readfirstlane(pages_lds[page_key0 / kPage]) * kPage;
      row_last = (int64_t)__builtin_amdgcn_readfirstlane(pages_lds[kv_last / kPage]) * kPage +
                 kv_last % kPage;
    }
    const uint8_t* base = reinterpret_cast<const uint8_t*>(v ? vbase : kbase);
    const uint8_t* src = base + row0 * kv_row * 2;
    const uint8_t* src_last = base + row_last * kv_row * 2;
#pragma unroll
    for (int j = 0; j < SLABS; ++j) {
      const int slab = wave * SLABS + j;
      const int key = slab * KEYS_PER_SLAB + lane / KCH;  // within the tile
      const int p = lane % KCH;
      const uint32_t chunk = (uint32_t)((p ^ (v ? vswz<D>(key) : kswz<D>(key))) * 16);
      const uint8_t* at = t * kBK + key < kv_end ? src + (v ? voff[j] : koff[j]) : src_last + chunk;
      lds_dma16(at, (v ? v_buf(buf) : k_buf(buf)) + slab * 1024);
    }
  };

  // lane-constant parts of the LDS read addresses
  // K fragment (A operand of S^T): key `col` (+32 for the second subtile),
  // d chunk 2c + half
  int k_off[ND16];
#pragma unroll
  for (int c = 0; c < ND16; ++c) k_off[c] = col * ROW + (((2 * c + half) ^ kswz<D>(col)) * 16);
  // V^T fragment (A operand of O^T) by transposing reads: lane 16g + x reads
  // 4 halfwords of key 4*half + x/4 (+8 for the second read) at d offset
  // 16*(g&1) + 4*(x&3) within each 32-d tile
  int v_off[NDS];
  {
    const int x = lane & 15;
    const int key_rel = 4 * half + (x >> 2);
    const int chunk = 2 * ((lane >> 4) & 1) + ((x & 3) >> 1);
#pragma unroll
    for (int dt = 0; dt < NDS; ++dt)
      v_off[dt] = key_rel * ROW + (((dt * 4 + chunk) ^ vswz<D>(key_rel)) * 16) + 8 * (x & 1);
  }

  v16f o[NDS];
#pragma unroll
  for (int d = 0; d < NDS; ++d)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[d][e] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  const int lim = causal ? min(off + r + 1, used_s) : used_s;  // keys < lim are visible
  // the smallest visible-key limit over this wave's rows, and whether all 32
  // of its rows are real: tiles below that limit skip the mask
  const int wave_first = qt * BQ + qsub * 32;
  const int wave_lim_min = causal ? min(off + wave_first + 1, used_s) : used_s;
  const bool wave_rows_full = wave_first + 32 <= q_len;

  // Software pipeline over KV tiles, two LDS buffers each for K and V.
  // Step t computes S of tile t + 1 (K buffer (t+1)%2) in the same basic
  // block as the softmax and PV of tile t (V buffer t%2), so the S MFMAs of
  // one tile overlap the VALU work of the previous one; meanwhile K of tile
  // t + 2 and V of tile t + 1 load into the buffers steps t - 2 and t - 1
  // released. Tiles past this wave's rows are fully masked (they add
  // nothing); tiles past the last are neither loaded nor computed.
  auto s_tile = [&](const int buf, v16f (&sacc)[2]) {
    const uint8_t* kl = k_buf(buf);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) sacc[ks] = v16f{};
#pragma unroll
    for (int c = 0; c < ND16; ++c)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const v8s kf = *reinterpret_cast<const v8s*>(kl + ks * 32 * ROW + k_off[c]);
        sacc[ks] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            __builtin_bit_cast(v8bf, kf), __builtin_bit_cast(v8bf, qf[c]), sacc[ks], 0, 0, 0);
      }
  };
  auto mask_tile = [&](const int t, v16f (&sacc)[2]) {
    // a tile every row of this wave sees whole needs no mask (wave-uniform)
    const int t0 = t * kBK;
    if (t0 + kBK <= wave_lim_min && wave_rows_full) return;
    // key (ks, i) of this lane is t0 + half * 4 + ks * 32 + (i / 4) * 8 + i % 4:
    // visible when that constant offset is below `room` (none for a padding row)
    const int room = r_ok ? lim - t0 - half * 4 : -1;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int i = 0; i < 16; ++i)
        sacc[ks][i] = ks * 32 + (i >> 2) * 8 + (i & 3) < room ? sacc[ks][i] : -INFINITY;
  };
  auto softmax_pv = [&](const int buf, v16f (&sacc)[2]) {
    // the running max is kept on raw scores (scale_log2 > 0), and the scale
    // folds into one fma per score: p = exp2(s * scale_log2 - m * scale_log2)
    float tmax = -INFINITY;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int i = 0; i < 16; ++i) tmax = fmaxf(tmax, sacc[ks][i]);
    tmax = max_halves(tmax);
    // Lazy rescale: the reference max m_run, against which p and O are kept,
    // moves only when a tile raises the row max by more than kLazyLog2 (log2
    // units, so p < 2^kLazyLog2), and O is rescaled only
    // when some row of the wave moved: VALU work on the MFMA accumulators
    // stalls the matrix core, and after a row's first tiles its max rarely
    // jumps that far. A tile that adds nothing to a row (wholly masked for
    // it, max -inf) never moves it and leaves its state bit for bit, so a
    // row's result does not depend on how many such tiles its workgroup
    // visits. (m_cand - m_run is NaN, so "no move", while both are -inf.)
    const float m_cand = fmaxf(m_run, tmax);
    const bool move = (m_cand - m_run) * scale_log2 > kLazyLog2;
    const float alpha = move ? __builtin_amdgcn_exp2f((m_run - m_cand) * scale_log2) : 1.0f;
    m_run = move ? m_cand : m_run;
    const float m_use = m_run == -INFINITY ? 0.f : m_run * scale_log2;
    if (__builtin_amdgcn_ballot_w64(move)) {  // wave-uniform; alpha is 1 where a row did not move
#pragma unroll
      for (int d = 0; d < NDS; ++d)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[d][e] *= alpha;
    }
    float psum = 0.f;
    using PV = std::conditional_t<VBF, v8bf, v8h>;
    PV pf[4];
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        // arguments are <= kLazyLog2, inside v_exp_f32's range
        const float pv =
            __builtin_amdgcn_exp2f(fmaf(sacc[kc >> 1][(kc & 1) * 8 + j], scale_log2, -m_use));
        psum += pv;
        if constexpr (VBF) {
          pf[kc][j] = (__bf16)pv;
        } else {
          pf[kc][j] = (_Float16)pv;
        }
      }
    }
    psum = sum_halves(psum);
    l_run = l_run * alpha + psum;

    // O^T += V^T P^T: MFMA kc covers keys kc/2*32 + (kc&1)*16 +
    // {4*half + 0..3, 8 + 4*half + 0..3} in its k slots half*8 + 0..7, the
    // order in which P^T's lanes hold them
    const uint8_t* vl = v_buf(buf);
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
      const int kbase_b = ((kc >> 1) * 32 + (kc & 1) * 16) * ROW;
      PV vf[NDS];
#pragma unroll
      for (int d = 0; d < NDS; ++d) {
        const v4s lo =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(vl + kbase_b + v_off[d]));
        const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_v4s*)(vl + kbase_b + 8 * ROW + v_off[d]));
        const v8s both = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        vf[d] = __builtin_bit_cast(PV, both);
      }
#pragma unroll
      for (int d = 0; d < NDS; ++d)
        if constexpr (VBF) {
          o[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[d], pf[kc], o[d], 0, 0, 0);
        } else {
          o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[d], pf[kc], o[d], 0, 0, 0);
        }
    }
  };

  v16f sa[2], sb[2];
  // prologue: K and V of tile 0 and K of tile 1 (with q-norm on load, Q's
  // norm and RoPE while they and the cos / sin rows are in flight), then S
  // of tile 0
  if (ntiles > 0) {
    issue(0, 0, false);
    issue(0, 0, true);
    if (ntiles > 1) issue(1, 1, false);
  }
  if constexpr (QN != 0) q_norm_rope_apply(qf, qin, qn.eps);
  if (ntiles > 0) {
    wait_vmcnt<0>();
    lds_barrier();
    s_tile(0, sa);
    lds_barrier();  // every wave has read K of tile 0 before step 0 reloads its buffer
  }
  // one step; `cur` (the parity of t) is a literal at both call sites
  // (the loads and the S of tiles past the last are skipped: wave-uniform
  // branches, 5-8% faster than computing them from stale data)
  auto step = [&](const int t, const int cur, v16f (&s_cur)[2], v16f (&s_next)[2]) {
    if (t + 2 < ntiles) issue(t + 2, cur, false);    // K buffer of tile t, read by step t - 1
    if (t + 1 < ntiles) issue(t + 1, cur ^ 1, true);  // V buffer of tile t - 1, read by step t - 1
    mask_tile(t, s_cur);
    if (t + 1 < ntiles) s_tile(cur ^ 1, s_next);      // K of tile t + 1, loaded during step t - 1
    softmax_pv(cur, s_cur);
    wait_vmcnt<0>();  // this wave's loads of this step landed
    lds_barrier();
  };
  for (int t = 0; t < ntiles; t += 2) {
    step(t, 0, sa, sb);
    if (t + 1 < ntiles) step(t + 1, 1, sb, sa);
  }

  // ---- epilogue: lane holds query `col`, d = dt*32 + (i/4)*8 + half*4 + i%4
  const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
  const int64_t row = q0 + r;
  if (lse && r_ok && half == 0) {
    // p was kept against m_run: ln(sum exp(scale * s)) = ln 2 * (log2 l + m_run * scale_log2)
    const float m_use = m_run == -INFINITY ? 0.f : m_run * scale_log2;
    lse[(int64_t)head * lse_ld + row] =
        l_run > 0.f ? (__log2f(l_run) + m_use) * 0.6931471805599453f : -INFINITY;
  }
  // The wave's 32 output rows go out through LDS (the K/V buffers: after
  // the last step's barrier every wave's loads have landed and its reads of
  // them are consumed) so that each global store writes whole rows: from
  // the MFMA layout a lane holds 4-value runs of one row, and every store
  // instruction would touch 32 rows.
  // LDS rows hold their 16-byte chunks XOR-swizzled by the row (chunk
  // c of row rr at c ^ (rr % CH)), which spreads a store's 32 rows over
  // the banks without padding
  constexpr int OUT_BYTES = QUANT ? D : 2 * D;  // bytes of one head's row
  constexpr int CH = OUT_BYTES / 16;            // 16-byte chunks per row
  static_assert(NW * 32 * OUT_BYTES <= 2 * 2 * T_BYTES, "epilogue staging");
  uint8_t* stage = &kv_lds[0][0][0] + wave * 32 * OUT_BYTES;
  // byte b of row rr in the staged tile
  auto slot = [&](int rr, int b) { return rr * OUT_BYTES + (((b >> 4) ^ (rr % CH)) << 4) + (b & 15); };
  const int wave_row0 = qt * BQ + qsub * 32;         // the wave's first row in the sequence
  const int rows_here = min(32, q_len - wave_row0);  // of which exist
  if (QUANT) {
    float amax = 0.f;
#pragma unroll
    for (int d = 0; d < NDS; ++d)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float v = round_bf16(o[d][e] * inv);
        o[d][e] = v;
        amax = fmaxf(amax, fabsf(v));
      }
    amax = max_halves(amax);
    const float sc = fp8_scale(amax);
    const float rsc = recip(sc);
#pragma unroll
    for (int d = 0; d < NDS; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int dd = d * 32 + g * 8 + half * 4;
        *reinterpret_cast<uint32_t*>(stage + slot(col, dd)) =
            pack4_fp8(div_by(o[d][g * 4], sc, rsc), div_by(o[d][g * 4 + 1], sc, rsc),
                      div_by(o[d][g * 4 + 2], sc, rsc), div_by(o[d][g * 4 + 3], sc, rsc));
      }
    if (r_ok && half == 0) scales[(int64_t)head * s_ld + row] = sc;
  } else {
#pragma unroll
    for (int d = 0; d < NDS; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int dd = d * 32 + g * 8 + half * 4;
        *reinterpret_cast<uint2*>(stage + slot(col, 2 * dd)) =
            make_uint2(pack2_bf16(o[d][g * 4] * inv, o[d][g * 4 + 1] * inv),
                       pack2_bf16(o[d][g * 4 + 2] * inv, o[d][g * 4 + 3] * inv));
      }
  }
  // the wave reads back what its other lanes wrote
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  constexpr int RPP = 64 / CH;  // rows per store instruction
  uint8_t* obase = QUANT ? out8 : reinterpret_cast<uint8_t*>(out16);
  const int64_t orow_bytes = QUANT ? o_ld : 2 * o_ld;
#pragma unroll
  for (int pass = 0; pass < 32 / RPP; ++pass) {
    const int rr = pass * RPP + lane / CH;
    const int ch = lane % CH;
    const v4i val = *reinterpret_cast<const v4i*>(stage + slot(rr, ch * 16));
    if (rr < rows_here)
      *reinterpret_cast<v4i*>(obase + (int64_t)(q0 + wave_row0 + rr) * orow_bytes +
                              head * OUT_BYTES + ch * 16) = val;
  }
}

template <int D, int HPB, int QSUB, bool VBF>
int launch_attn_v(const void* q, int64_t q_ld, const int64_t* q_index, const void* kp,
                  const void* vp, const int* cu_q, const int* used, const int* table,
                  int64_t table_ld, const int* cu_k, int seqs, int max_q, int max_used, int HQ,
                  int HK, int page, float scale, int causal, void* out16, void* out8,
                  int64_t o_ld, float* scales, int64_t s_ld, float* lse, int64_t lse_ld,
                  const int* work, int n_work, const QNormArgs* qn, int qn_f32,
                  hipStream_t stream) {
  const int G = HQ / HK;
  constexpr int BQ = 32 * QSUB;
  const int zgroups = HK * (G / HPB);
  dim3 grid = work ? dim3((unsigned)n_work * zgroups, 1, 1)
                   : dim3((max_q + BQ - 1) / BQ, seqs, zgroups);
  const float scale_log2 = scale * 1.4426950408889634f;
  const dim3 block(HPB * QSUB * 64);
  const uint16_t* q16 = (const uint16_t*)q;
  const uint16_t* k16 = (const uint16_t*)kp;
  const uint16_t* v16 = (const uint16_t*)vp;
  bool launched = false;
  if constexpr (D == 128) {
    if (out8 && qn) {
      if (qn_f32)
        hipLaunchKernelGGL((paged_attention_kernel<D, HPB, QSUB, true, false, VBF, 2>), grid,
                           block, 0, stream, q16, q_ld, q_index, k16, v16, cu_q, used, table,
                           table_ld, cu_k, max_used, HQ, HK, scale_log2, causal, nullptr,
                           (uint8_t*)out8, o_ld, scales, s_ld, lse, lse_ld, work, zgroups, seqs,
                           *qn);
      else
        hipLaunchKernelGGL((paged_attention_kernel<D, HPB, QSUB, true, false, VBF, 1>), grid,
                           block, 0, stream, q16, q_ld, q_index, k16, v16, cu_q, used, table,
                           table_ld, cu_k, max_used, HQ, HK, scale_log2, causal, nullptr,
                           (uint8_t*)out8, o_ld, scales, s_ld, lse, lse_ld, work, zgroups, seqs,
                           *qn);
      launched = true;
    }
  }
  if (launched) {
  } else if (out8) {
    hipLaunchKernelGGL((paged_attention_kernel<D, HPB, QSUB, true, false, VBF>), grid, block, 0,
                       stream, q16, q_ld, q_index, k16, v16, cu_q, used, table, table_ld, cu_k,
                       max_used, HQ, HK, scale_log2, causal, nullptr, (uint8_t*)out8, o_ld,
                       scales, s_ld, lse, lse_ld, work, zgroups, seqs, QNormArgs{});
  } else if (cu_k) {
    hipLaunchKernelGGL((paged_attention_kernel<D, HPB, QSUB, false, true, VBF>), grid, block, 0,
                       stream, q16, q_ld, q_index, k16, v16, cu_q, used, table, table_ld, cu_k,
                       max_used, HQ, HK, scale_log2, causal, (uint16_t*)out16, nullptr, o_ld,
                       nullptr, 0, lse, lse_ld, work, zgroups, seqs, QNormArgs{});
  } else {
    hipLaunchKernelGGL((paged_attention_kernel<D, HPB, QSUB, false, false, VBF>), grid, block, 0,
                       stream, q16, q_ld, q_index, k16, v16, cu_q, used, table, table_ld, cu_k,
                       max_used, HQ, HK, scale_log2, causal, (uint16_t*)out16, nullptr, o_ld,
                       nullptr, 0, lse, lse_ld, work, zgroups, seqs, QNormArgs{});
  }
  QX_LAUNCH_STATUS();
}

template <int D, int HPB, int QSUB>
int launch_attn(const void* q, int64_t q_ld, const int64_t* q_index, const void* kp,
                const void* vp, const int* cu_q, const int* used, const int* table,
                int64_t table_ld, const int* cu_k, int seqs, int max_q, int max_used, int HQ,
                int HK, int page, float scale, int causal, void* out16, void* out8, int64_t o_ld,
                float* scales, int64_t s_ld, float* lse, int64_t lse_ld, const int* work,
                int n_work, int v_bf16, const QNormArgs* qn, int qn_f32, hipStream_t stream) {
  if (v_bf16)
    return launch_attn_v<D, HPB, QSUB, true>(q, q_ld, q_index, kp, vp, cu_q, used, table,
                                             table_ld, cu_k, seqs, max_q, max_used, HQ, HK, page,
                                             scale, causal, out16, out8, o_ld, scales, s_ld, lse,
                                             lse_ld, work, n_work, qn, qn_f32, stream);
  return launch_attn_v<D, HPB, QSUB, false>(q, q_ld, q_index, kp, vp, cu_q, used, table,
                                            table_ld, cu_k, seqs, max_q, max_used, HQ, HK, page,
                                            scale, causal, out16, out8, o_ld, scales, s_ld, lse,
                                            lse_ld, work, n_work, qn, qn_f32, stream);
}

// The tree path's merge (attention.py:902-948, merge_attn_quant with QUANT):
// row t's result from call A (its own segment) and, when source[t] >= 0,
// row source[t] of call B (its reads of resident pages) are combined by
// their log-sum-exps, w = bf16(sigmoid(lse_b - lse_a)),
// y = bf16(a + (b - a) * w), and y is quantized per head to e4m3 with
// scale max(amax, 1e-10) / 448, as the o_proj input (QUANT, D = 128), or
// stored as bf16 (QUANT off). One wave per (row, 512 columns): each lane
// Call C's merge into call B's rows (merge_partial, attention.py:407-429):
// one wave per (i, head); row index[i] of out / lse takes
// out*wb/(wb+wc) + out_c*wc/(wb+wc) with wb = exp(lb - top), wc = exp(lc - top),
// top = max(lb, lc), and lse top + ln(wb + wc); a pair with no keys on
// either side (top = -inf) is left as it is.
__global__ __launch_bounds__(256) void merge_partial_kernel(
    uint16_t* __restrict__ out, int64_t o_ld, float* __restrict__ lse, int64_t l_ld,
    const int64_t* __restrict__ index, const uint16_t* __restrict__ oc, int64_t c_ld,
    const float* __restrict__ lc, int64_t lc_ld, int count, int H, int D) {
  const int lane = threadIdx.x & 63;
  const int wid = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wid >= count * H) return;
  const int i = wid / H;
  const int h = wid % H;
  const int64_t r = index[i];
  const float b = lse[h * l_ld + r];
  const float c = lc[h * lc_ld + i];
  const float top = fmaxf(b, c);
  if (top == -INFINITY) return;
  const float wb = expf(b - top), wc = expf(c - top);
  const float total = wb + wc;
  const float fb = wb / total, fc = wc / total;
  uint16_t* orow = out + r * o_ld + h * D;
  const uint16_t* crow = oc + (int64_t)i * c_ld + h * D;
  for (int e = lane; e < D; e += 64) {
    const float y = bf16_to_f32(orow[e]) * fb + bf16_to_f32(crow[e]) * fc;
    orow[e] = f32_to_bf16(y);
  }
  if (lane == 0) lse[h * l_ld + r] = top + logf(total);
}

// holds 8 consecutive values of one head.
template <bool QUANT>
__global__ __launch_bounds__(256) void merge_attn_quant_kernel(
    const uint16_t* __restrict__ a, int64_t a_ld, const uint16_t* __restrict__ b, int64_t b_ld,
    const float* __restrict__ la, int64_t la_ld, const float* __restrict__ lb, int64_t lb_ld,
    const int* __restrict__ source, uint8_t* __restrict__ q, int64_t q_ld,
    float* __restrict__ scales, int64_t s_ld, int n, int width, int blocks, int D) {
  const int lane = threadIdx.x & 63;
  const int wid = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wid >= n * blocks) return;
  const int row = wid / blocks;
  const int col = (wid % blocks) * 512 + lane * 8;
  if (col >= width) return;  // whole heads leave together
  const int head = col / D;
  const int src = source[row];
  float y[8];
  const uint4 av = *reinterpret_cast<const uint4*>(a + (int64_t)row * a_ld + col);
  const uint32_t aw[4] = {av.x, av.y, av.z, av.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    y[2 * k] = lo_bf16(aw[k]);
    y[2 * k + 1] = hi_bf16(aw[k]);
  }
  if (src >= 0) {
    const float x = lb[(int64_t)head * lb_ld + src] - la[(int64_t)head * la_ld + row];
    const float w = round_bf16(1.0f / (1.0f + expf(-x)));
    const uint4 bv = *reinterpret_cast<const uint4*>(b + (int64_t)src * b_ld + col);
    const uint32_t bw[4] = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      y[2 * k] = round_bf16(fmaf(lo_bf16(bw[k]) - y[2 * k], w, y[2 * k]));
      y[2 * k + 1] = round_bf16(fmaf(hi_bf16(bw[k]) - y[2 * k + 1], w, y[2 * k + 1]));
    }
  }
  if (!QUANT) {
    uint4 o;
    o.x = pack2_bf16(y[0], y[1]);
    o.y = pack2_bf16(y[2], y[3]);
    o.z = pack2_bf16(y[4], y[5]);
    o.w = pack2_bf16(y[6], y[7]);
    *reinterpret_cast<uint4*>(q + ((int64_t)row * q_ld + col) * 2) = o;
    return;
  }
  float amax = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) amax = fmaxf(amax, fabsf(y[k]));
  amax = group_max<16>(amax);
  const float scale = fp8_scale(amax);
  const float rs = recip(scale);
  uint2 o;
  o.x = pack4_fp8(div_by(y[0], scale, rs), div_by(y[1], scale, rs), div_by(y[2], scale, rs),
                  div_by(y[3], scale, rs));
  o.y = pack4_fp8(div_by(y[4], scale, rs), div_by(y[5], scale, rs), div_by(y[6], scale, rs),
                  div_by(y[7], scale, rs));
  *reinterpret_cast<uint2*>(q + (int64_t)row * q_ld + col) = o;
  if ((lane & 15) == 0) scales[(int64_t)head * s_ld + row] = scale;
}

// Query heads per workgroup for (G = HQ / HK): the largest of 4, 2, 1
// dividing G.
inline int attn_heads_per_group(int64_t G) { return G % 4 == 0 ? 4 : (G % 2 == 0 ? 2 : 1); }

// Query rows per workgroup (work-list tile height) of a call: by default
// 32 * QSUB with HPB * QSUB = 8 waves, one workgroup per CU; with D = 128 and
// 4 heads per workgroup also 32 (4 waves, two workgroups per CU, which hide
// each other's fixed cost on short documents).
inline int attn_default_rows(int64_t G) { return 32 * (8 / attn_heads_per_group(G)); }
inline bool attn_rows_ok(int64_t D, int64_t G, int64_t rows) {
  return rows == attn_default_rows(G) || (D == 128 && attn_heads_per_group(G) == 4 && rows == 32);
}

// The 32-row tile is chosen when a pack's 64-row work items read at most
// this many 64-key tiles on average (measured crossover on MI355X: 768-token
// documents, 7.5 tiles per item, run 1.5% faster with it, 1024-token ones,
// 9.5 tiles, 1.2% slower).
constexpr double kShortItemTiles = 8.0;

}  // namespace
}  // namespace qx

namespace qx {
namespace {

int attention_impl(const void* q, int64_t q_ld, const int64_t* q_index, const void* k_pool,
                   const void* v_pool, const int* cu_q, const int* used, const int* table,
                   int64_t table_ld, const int* cu_k, int64_t seqs, int64_t max_q,
                   int64_t max_used, int64_t HQ, int64_t HK, int64_t D, int64_t page, float scale,
                   int causal, void* out_bf16, void* out_fp8, int64_t o_ld, float* scales,
                   int64_t s_ld, float* lse, int64_t lse_ld, const int* work, int64_t n_work,
                   int64_t tile_rows, int v_bf16, hipStream_t stream,
                   const QNormArgs* qn = nullptr, int qn_f32 = 0) {
  QX_CHECK(q && k_pool && v_pool && cu_q && used && (table || cu_k), "attention: null pointer");
  QX_CHECK(out_bf16 || out_fp8, "attention: no output");
  QX_CHECK(!(out_fp8 && (cu_k || lse || q_index)), "attention: fused quant is for the paged call");
  QX_CHECK(D == 64 || D == 128, "attention: head_dim %lld", (long long)D);
  QX_CHECK(HQ > 0 && HK > 0 && HQ % HK == 0, "attention: heads %lld/%lld", (long long)HQ,
           (long long)HK);
  QX_CHECK(page == kPage, "attention: page of %lld tokens (the arena uses 16)", (long long)page);
  QX_CHECK(max_used >= 0 && (cu_k || max_used <= (int64_t)kMaxPages * page),
           "attention: max_used %lld exceeds %d pages", (long long)max_used, kMaxPages);
  QX_CHECK(q_ld % 8 == 0 && o_ld % 4 == 0, "attention: strides");
  QX_CHECK(!out_fp8 || (D == 128 && scales), "attention: fused quant needs D=128 and scales");
  QX_CHECK(seqs < 65536, "attention: %lld sequences exceed the grid", (long long)seqs);
  QX_CHECK(!work || (n_work >= 0 && n_work * HK * 8 < (1LL << 31)), "attention: work items");
  const int G = (int)(HQ / HK);
  const int hpb = attn_heads_per_group(G);
  const int64_t rows = tile_rows ? tile_rows : attn_default_rows(G);
  QX_CHECK(attn_rows_ok(D, G, rows), "attention: %lld query rows per workgroup (D=%lld, G=%d)",
           (long long)rows, (long long)D, G);
  if (seqs == 0 || max_q == 0 || (work && n_work == 0)) return QX_OK;
  const int args_seqs = (int)seqs, args_mq = (int)max_q, args_mu = (int)max_used;
#define QX_ATTN(DD, HPB_, QS_)                                                                 \
  return launch_attn<DD, HPB_, QS_>(q, q_ld, q_index, k_pool, v_pool, cu_q, used, table,       \
                                    table_ld, cu_k, args_seqs, args_mq, args_mu, (int)HQ,      \
                                    (int)HK, (int)page, scale, causal, out_bf16, out_fp8,      \
                                    o_ld, scales, s_ld, lse, lse_ld, work, (int)n_work,        \
                                    v_bf16, qn, qn_f32, stream)
  if (D == 128) {
    if (hpb == 4 && rows == 32) QX_ATTN(128, 4, 1);
    if (hpb == 4) QX_ATTN(128, 4, 2);
    if (hpb == 2) QX_ATTN(128, 2, 4);
    QX_ATTN(128, 1, 8);
  } else {
    if (hpb == 4) QX_ATTN(64, 4, 2);
    if (hpb == 2) QX_ATTN(64, 2, 4);
    QX_ATTN(64, 1, 8);
  }
#undef QX_ATTN
}

}  // namespace
}  // namespace qx

extern "C" {


// The most keys one sequence of a paged call may see: the page-table row a
// workgroup stages in LDS holds kMaxPages entries.
int64_t qx_paged_attention_max_keys(int64_t page) {
  if (page != qx::kPage) {
    qx::set_error("attention: page of %lld tokens (the arena uses 16)", (long long)page);
    return -1;
  }
  return (int64_t)qx::kMaxPages * page;
}

// out_fp8 != NULL: write the e4m3 o_proj input and its scales (D must be
// 128); otherwise write bf16 to out_bf16. o_ld is in elements of the output.
// v_bf16: the V pool holds bf16 (the reference arena's pools), else fp16.
// max_used bounds every used[s] (FA's max_seqlen_k) and must be at most
// 2048 * page (the page-table row each workgroup stages in LDS).
int qx_paged_attention(const void* q, int64_t q_ld, const void* k_pool, const void* v_pool,
                       const int* cu_q, const int* used, const int* table, int64_t table_ld,
                       int64_t seqs, int64_t max_q, int64_t max_used, int64_t HQ, int64_t HK,
                       int64_t D, int64_t page, float scale, int causal, void* out_bf16,
                       void* out_fp8, int64_t o_ld, float* scales, int64_t s_ld,
                       const int* work, int64_t n_work, int64_t tile_rows, int v_bf16,
                       hipStream_t stream) {
  QX_CHECK(table, "attention: null pointer");
  return qx::attention_impl(q, q_ld, nullptr, k_pool, v_pool, cu_q, used, table, table_ld,
                            nullptr, seqs, max_q, max_used, HQ, HK, D, page, scale, causal,
                            out_bf16, out_fp8, o_ld, scales, s_ld, nullptr, 0, work, n_work,
                            tile_rows, v_bf16, stream);
}

// qx_paged_attention with the o_proj quant on q as the qkv projection left
// it: q (qkv's first HQ*128 columns, rows of q_ld) is normalized and rotated
// per row as it is loaded (the qk-norm-rope pass then writes K and V only).
int qx_paged_attention_qnorm(const void* q, int64_t q_ld, const void* k_pool, const void* v_pool,
                             const int* cu_q, const int* used, const int* table,
                             int64_t table_ld, int64_t seqs, int64_t max_q, int64_t max_used,
                             int64_t HQ, int64_t HK, int64_t D, int64_t page, float scale,
                             int causal, void* out_fp8, int64_t o_ld, float* scales, int64_t s_ld,
                             const int* work, int64_t n_work, int64_t tile_rows, int v_bf16,
                             const int64_t* positions, const void* cos_sin, int cs_is_f32,
                             const void* q_w, float eps, hipStream_t stream) {
  QX_CHECK(table && out_fp8 && scales && positions && cos_sin && q_w,
           "attention_qnorm: null pointer");
  QX_CHECK(D == 128, "attention_qnorm: head_dim %lld (128)", (long long)D);
  QX_CHECK(((uintptr_t)cos_sin & 15) == 0 && ((uintptr_t)q_w & 15) == 0,
           "attention_qnorm: cos_sin / q_w alignment");
  const qx::QNormArgs qn{positions, cos_sin, static_cast<const uint16_t*>(q_w), eps};
  return qx::attention_impl(q, q_ld, nullptr, k_pool, v_pool, cu_q, used, table, table_ld,
                            nullptr, seqs, max_q, max_used, HQ, HK, D, page, scale, causal,
                            nullptr, out_fp8, o_ld, scales, s_ld, nullptr, 0, work, n_work,
                            tile_rows, v_bf16, stream, &qn, cs_is_f32 ? 1 : 0);
}

// The tree path's two calls: bf16 output plus each row's log-sum-exp.
// table != NULL: paged keys as in qx_paged_attention; table == NULL: key j
// of sequence s is row cu_k[s] + j of k (bf16) and v, rows of HK * D
// elements. q_index (may be NULL): query row i reads Q row q_index[i].
// v_bf16: V (pool or rows) holds bf16, else fp16.
int qx_attention_lse(const void* q, int64_t q_ld, const int64_t* q_index, const void* k,
                     const void* v, const int* cu_q, const int* used, const int* table,
                     int64_t table_ld, const int* cu_k, int64_t seqs, int64_t max_q,
                     int64_t max_used, int64_t HQ, int64_t HK, int64_t D, float scale, int causal,
                     void* out_bf16, int64_t o_ld, float* lse, int64_t lse_ld, const int* work,
                     int64_t n_work, int v_bf16, hipStream_t stream) {
  QX_CHECK(out_bf16 && lse, "attention_lse: null output");
  QX_CHECK((table == nullptr) != (cu_k == nullptr), "attention_lse: give a table or cu_k");
  return qx::attention_impl(q, q_ld, q_index, k, v, cu_q, used, table, table_ld, cu_k, seqs,
                            max_q, max_used, HQ, HK, D, qx::kPage, scale, causal, out_bf16,
                            nullptr, o_ld, nullptr, 0, lse, lse_ld, work, n_work, 0, v_bf16,
                            stream);
}

// The tree path's LSE merge fused with the o_proj input quantization
// (attention.py:902-948): a (n, HQ*D) bf16 from the segment call with
// lse_a at la[h*la_ld + t], b (rows, HQ*D) bf16 from the resident-page call
// with lse_b at lb[h*lb_ld + j], source[t] = row of b for row t or -1.
// scales != NULL: writes e4m3 (n, HQ*D) to q and scales[h*s_ld + t]
// (D == 128, one quant group per head); scales == NULL: writes the bf16
// merge to q (q_ld in elements of either).
int qx_merge_attn_quant(const void* a, int64_t a_ld, const void* b, int64_t b_ld,
                        const float* la, int64_t la_ld, const float* lb, int64_t lb_ld,
                        const int* source, int64_t n, int64_t HQ, int64_t D, void* q,
                        int64_t q_ld, float* scales, int64_t s_ld, hipStream_t stream) {
  QX_CHECK(a && la && source && q, "merge_attn_quant: null pointer");
  QX_CHECK((D == 64 || D == 128) && HQ > 0, "merge_attn_quant: heads %lld x %lld",
           (long long)HQ, (long long)D);
  QX_CHECK(!scales || D == 128, "merge_attn_quant: the fused quant needs one head per group");
  QX_CHECK(a_ld % 8 == 0 && b_ld % 8 == 0 && q_ld % 8 == 0, "merge_attn_quant: strides");
  QX_CHECK(la_ld >= n && (!scales || s_ld >= n), "merge_attn_quant: lse / scale strides");
  if (n == 0) return QX_OK;
  const int width = (int)(HQ * D);
  const int blocks = (width + 511) / 512;
  const int64_t waves = n * blocks;
  const dim3 grid((unsigned)((waves + 3) / 4));
  if (scales) {
    hipLaunchKernelGGL(qx::merge_attn_quant_kernel<true>, grid, dim3(256), 0, stream,
                       (const uint16_t*)a, a_ld, (const uint16_t*)b, b_ld, la, la_ld, lb, lb_ld,
                       source, (uint8_t*)q, q_ld, scales, s_ld, (int)n, width, blocks, (int)D);
  } else {
    hipLaunchKernelGGL(qx::merge_attn_quant_kernel<false>, grid, dim3(256), 0, stream,
                       (const uint16_t*)a, a_ld, (const uint16_t*)b, b_ld, la, la_ld, lb, lb_ld,
                       source, (uint8_t*)q, q_ld, nullptr, 0, (int)n, width, blocks, (int)D);
  }
  QX_LAUNCH_STATUS();
}

int qx_merge_partial(void* out, int64_t o_ld, float* lse, int64_t lse_ld, const int64_t* index,
                     const void* out_c, int64_t c_ld, const float* lse_c, int64_t lse_c_ld,
                     int64_t count, int64_t H, int64_t D, hipStream_t stream) {
  QX_CHECK(out && lse && index && out_c && lse_c, "merge_partial: null pointer");
  QX_CHECK((D == 64 || D == 128) && H > 0, "merge_partial: heads %lld x %lld", (long long)H,
           (long long)D);
  QX_CHECK(o_ld >= H * D && c_ld >= H * D && lse_c_ld >= count, "merge_partial: strides");
  if (count == 0) return QX_OK;
  const int64_t waves = count * H;
  hipLaunchKernelGGL(qx::merge_partial_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0,
                     stream, (uint16_t*)out, o_ld, lse, lse_ld, index, (const uint16_t*)out_c,
                     c_ld, lse_c, lse_c_ld, (int)count, (int)H, (int)D);
  QX_LAUNCH_STATUS();
}

// Host function: the query rows per workgroup a paged call over these
// sequences runs best with (the tile height to build its work list and call
// it with): 32 where the configuration allows it and the 64-row work items
// read at most kShortItemTiles 64-key tiles on average, else the default.
int64_t qx_paged_attention_tile_rows(const int* cu_q, const int* used, int64_t seqs, int64_t HQ,
                                     int64_t HK, int64_t D, int causal) {
  if (!(cu_q && used && seqs >= 0 && HQ > 0 && HK > 0 && HQ % HK == 0)) {
    qx::set_error("attention_tile_rows: arguments");
    return QX_EINVAL;
  }
  const int64_t G = HQ / HK;
  const int bq = qx::attn_default_rows(G);
  if (!qx::attn_rows_ok(D, G, 32) || bq == 32) return bq;
  int64_t items = 0, tiles = 0;
  for (int64_t s = 0; s < seqs; ++s) {
    const int q_len = cu_q[s + 1] - cu_q[s];
    const int u = used[s];
    for (int qt = 0; qt * bq < q_len; ++qt) {
      const int last = std::min(qt * bq + bq, q_len) - 1;
      const int keys = causal ? std::min(u, u - q_len + last + 1) : u;
      tiles += (std::max(keys, 0) + 63) / 64;
      ++items;
    }
  }
  return items && (double)tiles <= qx::kShortItemTiles * (double)items ? 32 : bq;
}

// Host function: the work list of a paged call, one (sequence, query tile)
// item per query tile of tile_rows rows (0: the default for (HQ / HK, D))
// that holds rows, heaviest first (most keys to read; ties in sequence and
// tile order). Returns the number of items (<= capacity) or -1.
int64_t qx_paged_attention_work(const int* cu_q, const int* used, int64_t seqs, int64_t HQ,
                                int64_t HK, int64_t D, int causal, int64_t tile_rows, int* work,
                                int64_t capacity) {
  if (!(cu_q && used && work && seqs >= 0 && HQ > 0 && HK > 0 && HQ % HK == 0)) {
    qx::set_error("attention_work: arguments");
    return QX_EINVAL;
  }
  const int64_t G = HQ / HK;
  const int bq = (int)(tile_rows ? tile_rows : qx::attn_default_rows(G));
  if (!qx::attn_rows_ok(D, G, bq)) {
    qx::set_error("attention_work: %d query rows per workgroup (D=%lld, G=%lld)", bq,
                  (long long)D, (long long)G);
    return QX_EINVAL;
  }
  struct Item { int64_t load; int s, qt; };
  std::vector<Item> items;
  for (int64_t s = 0; s < seqs; ++s) {
    const int q_len = cu_q[s + 1] - cu_q[s];
    const int u = used[s];
    for (int qt = 0; qt * bq < q_len; ++qt) {
      const int last = std::min(qt * bq + bq, q_len) - 1;
      const int keys = causal ? std::min(u, u - q_len + last + 1) : u;
      items.push_back({(int64_t)keys, (int)s, qt});
    }
  }
  if ((int64_t)items.size() > capacity) {
    qx::set_error("attention_work: %zu items exceed the capacity %lld", items.size(),
                  (long long)capacity);
    return QX_EINVAL;
  }
  std::stable_sort(items.begin(), items.end(),
                   [](const Item& a, const Item& b) { return a.load > b.load; });
  for (size_t i = 0; i < items.size(); ++i) {
    work[2 * i] = items[i].s;
    work[2 * i + 1] = items[i].qt;
  }
  return (int64_t)items.size();
}

}  // extern "C"
