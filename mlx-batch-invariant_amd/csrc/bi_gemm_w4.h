// The 256 x 256 four-wave footprint of the batch-invariant GEMM (16-bit
// element types, 16-byte aligned operands), for outputs with many row blocks.
// Included by bi_gemm_kernel.h; it runs the same per-element chunk-step
// sequence as every other footprint (that file's header): chunk-step q is one
// v_mfma_f32_16x16x32_{bf16,f16} on k = 32q + 8g + t from lane group g, in
// ascending q, each accumulator starting at +0.0; the same epilogue.
//
// Shape. One workgroup of 4 waves, one per SIMD, owns a 256 x 256 tile of C;
// wave w owns the 128 x 128 sub-tile (w / 2, w % 2): 64 accumulator blocks of
// 16 x 16, held in AGPRs for the whole K loop (the MFMAs are inline asm tied
// to them, so no accumulator is ever copied). Per chunk-step a wave reads 8 A
// and 8 B operand chunks (16 KB per wave) for 64 MFMAs: half the LDS bytes
// per product of 64 x 64 wave tiles.
//
// Feed. A stage is 64 elements of K: 128 bytes of each of the 256 A rows and
// 256 B rows (or 64 k-rows of 512 bytes of a (K, N) B), so every load request
// is a whole 128-byte line. The LDS holds a ring of five 32 KB slots; stage s
// puts its A tile in slot (2s) % 5 and its B tile in slot (2s + 1) % 5. Loads
// go global -> LDS directly (buffer_load ... lds, 1 KB per instruction).
//
// Schedule, per stage s (chunk-steps 2s and 2s + 1; X_s is a workgroup
// barrier at the start of chunk-step 2s + 1):
//   chunk-step 2s:     64 MFMAs on operands in registers; between them the
//                      16 LDS reads of chunk-step 2s + 1 and the 8 loads of
//                      this wave's share of stage s + 2's A tile.
//   X_s:               this wave's loads of stage s + 1 have landed
//                      (vmcnt(8): only stage s + 2's A loads may be in
//                      flight), then the barrier: stage s + 1 is in LDS and
//                      nobody reads stage s any more.
//   chunk-step 2s + 1: 64 MFMAs; between them the reads of chunk-step
//                      2s + 2 (stage s + 1) and the loads of stage s + 2's
//                      B tile into the slot stage s's A tile freed.
// A tile gets three chunk-steps to land and a B tile two. The loads, LDS
// reads and MFMAs of a chunk-step are issued interleaved, instruction by
// instruction, so a load that waits for room in the memory pipeline holds up
// one MFMA slot, not a whole stage. Past K the tiles hold zeros (chunk-steps
// of exact zeros change no bit); the loop stops after stage ceil(K / 64) - 1.
#pragma once

namespace bi_gemm_dev {

template <typename T, bool TB>
struct W4Tile {
  static_assert(sizeof(T) == 2, "four-wave footprint: 16-bit element types");
  static constexpr int F = 8;          // 16 x 16 blocks per side of a wave's sub-tile
  static constexpr int WT = 16 * F;    // 128
  static constexpr int HALF = 32768;   // one operand tile of a stage, bytes
  static constexpr int EPS = 64;       // elements of K per stage
  static constexpr int NSLOT = 5;
  static constexpr int NDMA = 8;       // 1 KB loads per wave per operand tile
  static constexpr uint32_t kRowBytes = 128;  // bytes of an A row per stage

  f32x4_t acc[F][F];
  // Operand registers. B blocks and the last F - FA A blocks come in two
  // sets, alternating by chunk-step parity; A blocks below FA have one set,
  // each read again for the next chunk-step once its last MFMA is issued.
  static constexpr int FA = 6;
  u32x4_t av[FA], al[2][F - FA];
  u32x4_t bv[2][F];
  char* ring;                  // the LDS ring (generic pointer to __shared__ memory)
  uint32_t ring_lds;           // its LDS byte address
  int wave, lane;
  int64_t K, N;
  __amdgpu_buffer_rsrc_t ra, rb;
  // Operand reads: this lane's byte offset inside a slot of chunk-step j's
  // chunk of the wave's first 16-row block of A, of B (TB), or of B's 16-column
  // block jn ((K, N) B; chunk-step 1 is 32 k-rows on: +16384 bytes).
  uint32_t offa[2], offb[2], offbn[F];
  // Loads. A and (N, K) B: load i of this wave fills rows 32 i + 8 w +
  // lane / 8 of the slot, the lane's 16-byte chunk at position lane % 8 of the
  // row holding logical chunk (lane % 8) ^ (row % 8); ld_base is the byte
  // offset of that chunk in stage 0 for i = 0, ld_kidx its first K index,
  // ld_istep the bytes between rows 32 apart.
  uint32_t ld_base, ld_istep;
  int32_t ld_kidx;
  // (K, N) B: load i fills k-rows 8 i + 2 w + lane / 32, chunk lane % 32 of
  // the row holding logical chunk (lane % 32) ^ swz_nn(k-row) (which differs
  // between even and odd i); the offsets below are for stage 0 and i = 0 / 1.
  uint32_t nb_base[2];

  __device__ __forceinline__ void init(const GemmArgs& p, int64_t m0, int64_t n0) {
    constexpr int64_t E = 2;
    const int g = lane >> 4, r16 = lane & 15;
    const int wm = wave >> 1, wn = wave & 1;
    const T* A = static_cast<const T*>(p.a);
    const T* B = static_cast<const T*>(p.b);
    const int64_t M = p.M;
    ra = make_rsrc(A + m0 * K, min((int64_t)256, M - m0) * K * E);
    if constexpr (TB)
      rb = make_rsrc(B + n0 * K, min((int64_t)256, N - n0) * K * E);
    else
      rb = make_rsrc(B + n0, (K * N - n0) * E);
    // Operand reads (rows of 8 chunks, chunk c of row r at c ^ (r % 8)).
#pragma unroll
    for (int j = 0; j < 2; j++) {
      offa[j] = (uint32_t)((wm * WT + r16) * 8 + ((4 * j + g) ^ (r16 & 7))) * 16;
      offb[j] = (uint32_t)((wn * WT + r16) * 8 + ((4 * j + g) ^ (r16 & 7))) * 16;
    }
    if constexpr (!TB) {
      // As GemmTile::load_b: lane r16 of group g addresses k-row 8 g + r16 / 4
      // at column 4 (r16 % 4) of the block; the second 4 k-rows are +2048
      // bytes with the same swizzle.
#pragma unroll
      for (int jn = 0; jn < F; jn++) {
        const int kr = 8 * g + (r16 >> 2);
        const int col = wn * WT + jn * 16 + 4 * (r16 & 3);
        const int chunk = (col >> 3) ^ swz_nn<T, 32>(kr);
        offbn[jn] = (uint32_t)((kr * 32 + chunk) * 16 + (col & 7) * 2);
      }
    }
    // Loads of A (and of an (N, K) B): rows 8 w + lane / 8 (+ 32 i).
    {
      const int r = 8 * wave + (lane >> 3), c = (lane & 7) ^ (r & 7);
      ld_base = (uint32_t)(r * K * E + c * 16);
      ld_kidx = c * 8;
      ld_istep = (uint32_t)(32 * K * E);
    }
    if constexpr (!TB) {
#pragma unroll
      for (int par = 0; par < 2; par++) {
        const int kr = 8 * par + 2 * wave + (lane >> 5);
        const int c = (lane & 31) ^ swz_nn<T, 32>(kr);
        // A column outside N never loads.
        nb_base[par] = (n0 + c * 8 < N) ? (uint32_t)(kr * N * E + c * 16) : kOutOfRange;
      }
    }
  }

  __device__ __forceinline__ lds_void_t* slot_ptr(int slot, int i) const {
    return (lds_void_t*)(ring + slot * HALF + (i * 4 + wave) * 1024);
  }

  // Load i of this wave's share of the A tile of stage s (vo: the stage's
  // lane offset, or kOutOfRange past K).
  __device__ __forceinline__ void load_a(uint32_t vo, int slot, int i) const {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, slot_ptr(slot, i), 16, vo + i * ld_istep, 0, 0, 0);
  }
  __device__ __forceinline__ void load_b(uint32_t vo, int64_t s, int slot, int i) const {
    if constexpr (TB) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, slot_ptr(slot, i), 16, vo + i * ld_istep, 0, 0, 0);
    } else {
      // k-row 64 s + 8 i + ... (nb_base[i % 2] holds 8 (i % 2) of them):
      // rows at or past K lie outside rb; offsets that do not fit 31 bits
      // (far past K) load zeros too.
      const uint64_t o =
          (uint64_t)nb_base[i & 1] + (uint64_t)((s * EPS + 8 * (i & ~1)) * N * 2);
      const uint32_t off = o < kOutOfRange ? (uint32_t)o : kOutOfRange;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, slot_ptr(slot, i), 16, off, 0, 0, 0);
    }
  }
  __device__ __forceinline__ uint32_t stage_off(int64_t s) const {
    return ld_kidx + s * EPS < K ? ld_base + (uint32_t)(s * kRowBytes) : kOutOfRange;
  }

  template <int S>
  __device__ __forceinline__ void mfma(int k) {
    const int i = k >> 3, jn = k & 7;
    const u32x4_t& a = i < FA ? av[i] : al[S][i - FA];
    if constexpr (IsBF16<T>::value)
      asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0"
                   : "+a"(acc[i][jn]) : "v"(a), "v"(bv[S][jn]));
    else
      asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0"
                   : "+a"(acc[i][jn]) : "v"(a), "v"(bv[S][jn]));
  }

  // LDS byte address of this lane's operand chunk: slot base (a scalar) plus
  // the lane's offset, added in an asm statement so that the compiler keeps
  // one address register per read group instead of one per slot.
  __device__ __forceinline__ static uint32_t lds_at(uint32_t base, uint32_t off) {
    uint32_t a;
    asm volatile("v_add_u32 %0, %1, %2" : "=v"(a) : "s"(base), "v"(off));
    return a;
  }
  // A block i of the next chunk-step: blocks below FA into av, the last
  // F - FA into set S of al.
  template <int S>
  __device__ __forceinline__ void read_a(int i, uint32_t a) {
    if (i < FA)
      asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(av[i]) : "v"(a), "n"(i * 2048));
    else
      asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(al[S][i - FA]) : "v"(a), "n"(i * 2048));
  }
  // B block jn of chunk-step j into set S; `b` is the slot's address of the
  // lane's chunk (TB) or of block jn's first row ((K, N) B).
  template <int S>
  __device__ __forceinline__ void read_b(int jn, int j, uint32_t b) {
    if constexpr (TB) {
      asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(bv[S][jn]) : "v"(b), "n"(jn * 2048));
    } else {
      u32x2_t h0, h1;
      asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(h0) : "v"(b), "n"(j * 16384));
      asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(h1) : "v"(b), "n"(j * 16384 + 2048));
      bv[S][jn] = u32x4_t{h0.x, h0.y, h1.x, h1.y};
    }
  }

  // One chunk-step on operand set S: 64 MFMAs, block (i, jn) at position
  // 8 i + jn. Interleaved with them, the reads of the next chunk-step
  // (chunk-step j of the stage in slots nsa / nsb): its B blocks into set
  // 1 - S after MFMAs 0, 2, .., 14, its A blocks FA.. into set 1 - S of al
  // after MFMAs 16, 18, and each A block below FA right after the last MFMA
  // that reads it (after MFMA 8 i + 7), so the last read has 16 MFMAs to
  // land before the chunk-step's closing wait; and (LOAD: 1 = A tile, 2 = B
  // tile, 0 = none) this wave's 8 loads of stage s into slot dslot, after
  // MFMAs 8 d + 5.
  template <int S, int LOAD>
  __device__ __forceinline__ void chunk_step(int nj, int nsa, int nsb, uint32_t vo, int64_t s,
                                             int dslot) {
    const uint32_t abase = ring_lds + nsa * HALF, bbase = ring_lds + nsb * HALF;
    const uint32_t aaddr = lds_at(abase, offa[nj]);
    uint32_t baddr = 0;
    if constexpr (TB) baddr = lds_at(bbase, offb[nj]);
#pragma unroll
    for (int k = 0; k < 64; k++) {
      mfma<S>(k);
      if (k % 2 == 0 && k < 16) {
        if constexpr (TB)
          read_b<1 - S>(k / 2, nj, baddr);
        else
          read_b<1 - S>(k / 2, nj, lds_at(bbase, offbn[k / 2]));
      }
      if (k == 16 || k == 18) read_a<1 - S>(FA + (k - 16) / 2, aaddr);
      if (k % 8 == 7 && k / 8 < FA) read_a<1 - S>(k / 8, aaddr);
      if constexpr (LOAD == 1) {
        if (k % 8 == 5) load_a(vo, dslot, k / 8);
      } else if constexpr (LOAD == 2) {
        if (k % 8 == 5) load_b(vo, s, dslot, k / 8);
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }

  __device__ __forceinline__ static int mod5(int x) { return x >= NSLOT ? x - NSLOT : x; }

  // The K loop over nst stages. Stage s's A tile is in slot a = (2s) % 5,
  // its B tile in a + 1, stage s + 1's in a + 2 and a + 3, and stage s + 2's
  // A tile goes to a + 4 (the slot of stage s - 1's B tile), its B tile to a
  // (all mod 5).
  __device__ __forceinline__ void run(int64_t nst) {
#pragma unroll
    for (int i = 0; i < F; i++)
#pragma unroll
      for (int jn = 0; jn < F; jn++) acc[i][jn] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    // Prologue: stage 0's tiles and stage 1's A tile; then X_{-1} (stage 0
    // in LDS), stage 1's B tile, and chunk-step 0's operands.
    {
      const uint32_t v0 = stage_off(0), v1 = stage_off(1);
#pragma unroll
      for (int i = 0; i < NDMA; i++) load_a(v0, 0, i);
#pragma unroll
      for (int i = 0; i < NDMA; i++) load_b(v0, 0, 1, i);
#pragma unroll
      for (int i = 0; i < NDMA; i++) load_a(v1, 2, i);
      asm volatile("s_waitcnt vmcnt(8)\n\ts_barrier" ::: "memory");
#pragma unroll
      for (int i = 0; i < NDMA; i++) load_b(v1, 1, 3, i);
      const uint32_t aaddr = lds_at(ring_lds, offa[0]);
#pragma unroll
      for (int i = 0; i < F; i++) read_a<0>(i, aaddr);
      if constexpr (TB) {
        const uint32_t baddr = lds_at(ring_lds + HALF, offb[0]);
#pragma unroll
        for (int jn = 0; jn < F; jn++) read_b<0>(jn, 0, baddr);
      } else {
#pragma unroll
        for (int jn = 0; jn < F; jn++) read_b<0>(jn, 0, lds_at(ring_lds + HALF, offbn[jn]));
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    int a = 0;
    for (int64_t s = 0; s < nst; s++) {
      const uint32_t vo = stage_off(s + 2);
      // Chunk-step 2s: reads of chunk-step 2s + 1 (same stage), loads of
      // stage s + 2's A tile.
      chunk_step<0, 1>(1, a, mod5(a + 1), vo, s + 2, mod5(a + 4));
      // X_s.
      asm volatile("s_waitcnt vmcnt(8)\n\ts_barrier" ::: "memory");
      // Chunk-step 2s + 1: reads of chunk-step 2s + 2 (stage s + 1), loads
      // of stage s + 2's B tile.
      chunk_step<1, 2>(0, mod5(a + 2), mod5(a + 3), vo, s + 2, a);
      a = mod5(a + 2);
    }
    // No load may still be landing in the ring, and the last MFMA results
    // must be written before the accumulators are read (MFMA results are
    // not interlocked for plain VALU reads).
    asm volatile("s_waitcnt vmcnt(0)\n\ts_nop 15\n\ts_nop 15\n\ts_barrier" ::: "memory");
  }
};

template <typename T, bool TB>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
gemm_w4_kernel(GemmArgs p) {
  using Tile = W4Tile<T, TB>;
  constexpr int F = Tile::F, WT = Tile::WT;
  __shared__ uint4 ring[Tile::NSLOT * Tile::HALF / 16];
  Tile t;
  t.ring = reinterpret_cast<char*>(ring);
  t.ring_lds = (uint32_t)(uintptr_t)(lds_void_t*)ring;
  t.lane = threadIdx.x & 63;
  t.wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  t.K = p.K;
  t.N = p.N;
  const int tile = xcd_remap(blockIdx.x, p.tiles_m * p.tiles_n);
  int mi, ni;
  tile_coords(tile, p.tiles_m, p.tiles_n, mi, ni);
  const int64_t m0 = (int64_t)mi * 256, n0 = (int64_t)ni * 256;
  const int64_t M = p.M, N = p.N, K = p.K;
  t.init(p, m0, n0);
  t.run((K + Tile::EPS - 1) / Tile::EPS);

  // Epilogue (as gemm_kernel's): one rounding per element; whole sub-tiles
  // with 16-byte aligned output rows are rounded into slot `wave` of the ring
  // and stored as whole rows with 16-byte stores.
  const int g = t.lane >> 4, r16 = t.lane & 15;
  const int64_t wrow = m0 + (t.wave >> 1) * WT, wcol = n0 + (t.wave & 1) * WT;
  if (wrow >= M || wcol >= N) return;
  T* __restrict__ out = static_cast<T*>(p.out);
  const T* __restrict__ bias = static_cast<const T*>(p.bias);
  const float alpha = p.alpha, beta = p.beta;
  const bool whole = wrow + WT <= M && wcol + WT <= N && N % 8 == 0 &&
                     (reinterpret_cast<uintptr_t>(out) & 15) == 0;
  if (whole) {
    // Staging layout: element (r, c) of the sub-tile at byte
    // 256 r + 16 ((c / 8) ^ sw(r)) + 2 (c % 8), sw(r) = 2 ((r / 2) % 8).
    // Neighbouring lanes (columns c, c + 1 of one block) swap two rounded
    // values, so each lane writes two 4-byte pairs of columns: the even lane
    // rows 4g and 4g + 1, the odd lane rows 4g + 2 and 4g + 3. Either write of
    // the wave covers 8 rows of one 16-column block, 16 distinct 16-byte
    // chunks: every LDS bank once.
    char* stage = t.ring + t.wave * Tile::HALF;
    const uint32_t odd = -(uint32_t)(r16 & 1);  // all ones in odd lanes
    const int cp = r16 & ~1;  // first column of the lane's pair within the block
    const int rs = 2 * (r16 & 1);  // the lane's first row within its group of 4
#pragma unroll
    for (int jn = 0; jn < F; jn++) {
      const int c = jn * 16 + r16;
      const float bv = bias ? beta * Elem<T>::to_f32(bias[wcol + c]) : 0.f;
#pragma unroll
      for (int i = 0; i < F; i++) {
        uint32_t h[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
          float v = t.acc[i][jn][e];
          if (bias) v = __builtin_fmaf(alpha, v, bv);
          h[e] = __builtin_bit_cast(unsigned short, Elem<T>::from_f32(v));
        }
        // The even lane sends rows 2, 3 and keeps 0, 1; the odd lane the reverse.
        const uint32_t lo = h[0] | (h[1] << 16), hi = h[2] | (h[3] << 16);
        const uint32_t send = (hi & ~odd) | (lo & odd);
        const uint32_t got = (uint32_t)__builtin_amdgcn_mov_dpp((int)send, 0xb1, 0xf, 0xf, false);
        const uint32_t w0 = ((h[0] | (got << 16)) & ~odd) | (((got & 0xffffu) | (h[2] << 16)) & odd);
        const uint32_t w1 = ((h[1] | (got & 0xffff0000u)) & ~odd) | (((got >> 16) | (h[3] << 16)) & odd);
        const int r = i * 16 + 4 * g + rs;
        const int col = jn * 16 + cp;
        const int o0 = r * 256 + (((col >> 3) ^ (((r >> 1) & 7) << 1)) << 4) + (col & 7) * 2;
        const int o1 = (r + 1) * 256 + (((col >> 3) ^ ((((r + 1) >> 1) & 7) << 1)) << 4) + (col & 7) * 2;
        *reinterpret_cast<uint32_t*>(stage + o0) = w0;
        *reinterpret_cast<uint32_t*>(stage + o1) = w1;
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    // Rows back out as whole 256-byte rows: 16 lanes per row, 4 rows per pass.
    const int cc = t.lane & 15;
    T* orow = out + (wrow + (t.lane >> 4)) * N + wcol + cc * 8;
#pragma unroll
    for (int k = 0; k < WT / 4; k++) {
      const int r = 4 * k + (t.lane >> 4);
      const uint4 v = *reinterpret_cast<const uint4*>(stage + r * 256 + ((cc ^ (((r >> 1) & 7) << 1)) << 4));
      *reinterpret_cast<uint4*>(orow + 4 * k * N) = v;
    }
    return;
  }
#pragma unroll
  for (int jn = 0; jn < F; jn++) {
    const int64_t col = wcol + jn * 16 + r16;
    if (col >= N) continue;
    const float bv = bias ? beta * Elem<T>::to_f32(bias[col]) : 0.f;
#pragma unroll
    for (int i = 0; i < F; i++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int64_t row = wrow + i * 16 + 4 * g + e;
        if (row < M) {
          float v = t.acc[i][jn][e];
          if (bias) v = __builtin_fmaf(alpha, v, bv);
          out[row * N + col] = Elem<T>::from_f32(v);
        }
      }
  }
}

}  // namespace bi_gemm_dev
