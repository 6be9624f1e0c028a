// The quantized decode footprint of the batch-invariant GEMM: 2-, 4- and
// 8-bit affine weights, 16-bit activations, at most 8 rows of x. Included by
// bi_gemm_kernel.h; every element runs the quantized sequence of that file's
// quantized section: per group of K, P = the group's chunk-steps (ascending,
// the first from +0.0) of v_mfma_f32_16x16x32_{bf16,f16} on the x chunk and
// the codes as element-type integers, X the same on a chunk of ones; then, per
// group in ascending order, acc = fma(scale, P, acc) and acc = fma(bias, X,
// acc); one rounding at the end.
//
// Shape. A workgroup owns 16 output columns (every row: M <= MR <= 8) and NW
// waves. Groups are independent until their folds, so the waves split K
// instead of the columns: in a round of RK elements of K, wave w computes P
// and X of the groups in its BPW consecutive 128-element blocks and leaves
// them in LDS; after a barrier waves 0 .. GR - 1 fold the round's groups in
// ascending order, one output element per lane (wave w, lane 16 e + n: row
// 4 w + e, column n), and carry acc into the next round.
//
// Feed. All of a round's loads are issued at its start, in the order x,
// codes, scales and biases, so each wait lets the later loads stay in
// flight: a wave works on its first block of codes while the others land.
// x (rows 0 .. M - 1 of the round's K range) goes through registers into
// LDS, rows padded by 64 bytes so the rows' operand reads fall on distinct
// banks. Lane (g, n) of a wave reads the bytes of block b's codes of weight
// row n that hold chunk-step 4 b + g (16 bytes at 4 bits: four 32-bit words,
// one per lane group; 32 bytes at 8 bits: two words per lane group; 8 bytes at
// 2 bits: 16 bits per lane group, widened to a word each); a 4 x 4 transpose
// across the lane groups (two rounds of v_permlane32_swap /
// v_permlane16_swap; at 8 bits one for the even and one for the odd words)
// leaves in position j of lane group g its words of chunk-step 4 b + j -- the
// 8 codes of k = 32 q + 8 g + t, t = 0..7, the MFMA's B operand layout -- so
// every code load is whole 16-byte chunks (8 bytes at 2 bits) and no code
// passes through LDS.
#pragma once

namespace bi_gemm_dev {

template <int GS, int MR, int NW>
struct QDecode {
  static constexpr int RK = 4096;             // elements of K per round
  static constexpr int RG = RK / GS;          // groups per round
  static constexpr int CPG = GS / 32;         // chunk-steps per group
  static constexpr int NT = 64 * NW;
  static constexpr int BPW = RK / 128 / NW;   // blocks of 128 elements per wave per round
  static constexpr int XROW = RK * 2 + 64;    // bytes per staged row of x
  static constexpr int XPL = RK / 8 / NT;     // 16-byte x chunks per thread and row
  static constexpr int SRS = RG + 4;          // scale/bias row stride (f32), banks apart
  static constexpr int SPL = 16 * RG / NT;    // scale (and bias) entries per thread
  static_assert((RK / 8) % NT == 0 && (16 * RG) % NT == 0 && BPW >= 1, "round split");
  static_assert(GS >= 32 && GS <= 128, "groups of one to four chunk-steps: a block holds whole groups");
  static_assert(MR >= 1 && MR <= 8, "one to eight rows");
  // LDS: x rows; P of each group (rows 0 .. MR - 1, 16 columns, [row][column]);
  // X of each group (rows 0 .. 4 GR - 1); scales and biases as fp32, a row per
  // column; and 256 bytes that lanes with nothing to store write to instead
  // (so the stores need no branch; nothing reads them).
  static constexpr int GR = (MR + 3) / 4;     // lane groups whose MFMA rows are rows of x
  static constexpr int XS = 16 * GR;          // bytes of X per group
  static constexpr int OFF_P = MR * XROW;
  static constexpr int OFF_X = OFF_P + RG * MR * 64;
  static constexpr int OFF_S = OFF_X + RG * XS;
  static constexpr int OFF_Z = OFF_S + 16 * SRS * 4;
  static constexpr int OFF_DUMMY = OFF_Z + 16 * SRS * 4;
  static constexpr int LDS_BYTES = OFF_DUMMY + 256;
};

template <typename T, int GS, int MR, int NW, int QB>
__global__ void __launch_bounds__(64 * NW) gemm_qdecode_kernel(GemmArgs p) {
  static_assert(QB == 2 || QB == 4 || QB == 8, "2-, 4- or 8-bit codes");
  using D = QDecode<GS, MR, NW>;
  // Words of a chunk-step per lane group: 2-bit half a word (widened to one
  // below), 4-bit 1, 8-bit 2; code words a lane loads per block: 2, 4 or 8.
  constexpr int WPL = QB == 8 ? 2 : 1;
  constexpr int CW = QB == 8 ? 8 : QB == 4 ? 4 : 2;
  constexpr int RK = D::RK, RG = D::RG, CPG = D::CPG, BPW = D::BPW, NT = D::NT;
  constexpr int64_t E = 2;
  __shared__ __attribute__((aligned(16))) char lds[D::LDS_BYTES];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, r16 = lane & 15;
  const int64_t M = p.M, N = p.N, K = p.K;
  const int mrows = (int)M;  // 1 .. MR (the host checks)
  const int64_t n0 = (int64_t)blockIdx.x * 16;
  const int64_t G = K / GS;         // groups
  const int64_t nq = K / 32;        // chunk-steps
  const int64_t qrow = K * QB / 8;  // bytes of packed codes per weight row
  const int64_t cols = min((int64_t)16, N - n0);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.a, M * K * E);
  const __amdgpu_buffer_rsrc_t rw =
      make_rsrc(static_cast<const char*>(p.b) + n0 * qrow, cols * qrow);
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(static_cast<const T*>(p.qs) + n0 * G, cols * G * E);
  const __amdgpu_buffer_rsrc_t rz = make_rsrc(static_cast<const T*>(p.qz) + n0 * G, cols * G * E);

  // The A operand of chunk-step q of the round: lane (g, r) reads x row r at
  // k = 32 q + 8 g from the staged rows; rows past M read row 0 (an output
  // row depends only on its own row of x, and rows past M are not written).
  const uint32_t a_base = (uint32_t)((r16 < mrows ? r16 : 0) * D::XROW + 16 * g);
  constexpr uint32_t ONE = IsBF16<T>::value ? 0x3F803F80u : 0x3C003C00u;
  const uint4 ones = make_uint4(ONE, ONE, ONE, ONE);
  const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};

  float acc = 0.f;  // waves w < GR: element (row 4 w + lane / 16, column lane % 16)
  const int64_t rounds = (K + RK - 1) / RK;
  for (int64_t rr = 0; rr < rounds; rr++) {
    // The round index passes through an empty asm statement: nothing below
    // is then invariant across rounds, so the compiler hoists no address
    // arithmetic out of the loop (it would hold registers in every phase).
    int32_t r32 = (int32_t)rr;
    asm volatile("" : "+s"(r32));
    const int64_t r = r32;
    const int64_t k0 = r * RK;
    // Loads: x chunks of rows 0 .. M - 1 (the row of chunk i is the same for
    // every thread), this wave's blocks of codes, scale and bias entries.
    uint4 xv[MR][D::XPL];
#pragma unroll
    for (int row = 0; row < MR; row++)
#pragma unroll
      for (int i = 0; i < D::XPL; i++) {
        const int kc = tid + i * NT;
        const int64_t k = k0 + kc * 8;
        if (row < mrows) xv[row][i] = buffer_chunk(rx, k < K ? (uint32_t)((row * K + k) * E) : kOutOfRange);
      }
    // Lane (g, n) loads chunk-step 4 b + g's codes of weight row n: 16 bytes
    // at 4 bits, 32 at 8 (a 32-element chunk-step is 4 QB words of the row).
    uint32_t cw[BPW][CW];
#pragma unroll
    for (int j = 0; j < BPW; j++) {
      const int64_t q = (k0 >> 5) + 4 * (wave * BPW + j) + g;  // chunk-step this lane's bytes hold
      const uint32_t off = q < nq ? (uint32_t)(r16 * qrow + q * (4 * QB)) : kOutOfRange;
      if constexpr (QB == 2) {
        const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rw, (int)off, 0, 0));
        cw[j][0] = v.x;
        cw[j][1] = v.y;
      } else {
#pragma unroll
        for (int h = 0; h < CW / 4; h++) {
          const uint4 v = buffer_chunk(rw, off == kOutOfRange ? kOutOfRange : off + 16 * h);
          cw[j][4 * h + 0] = v.x;
          cw[j][4 * h + 1] = v.y;
          cw[j][4 * h + 2] = v.z;
          cw[j][4 * h + 3] = v.w;
        }
      }
    }
    unsigned short sv[D::SPL], zv[D::SPL];
#pragma unroll
    for (int i = 0; i < D::SPL; i++) {
      const int e = tid + i * NT, col = e / RG, gi = e % RG;
      const int64_t grp = r * RG + gi;
      const uint32_t off = grp < G ? (uint32_t)((col * G + grp) * E) : kOutOfRange;
      sv[i] = __builtin_amdgcn_raw_buffer_load_b16(rs, (int)off, 0, 0);
      zv[i] = __builtin_amdgcn_raw_buffer_load_b16(rz, (int)off, 0, 0);
    }
#pragma unroll
    for (int row = 0; row < MR; row++)
#pragma unroll
      for (int i = 0; i < D::XPL; i++) {
        const int kc = tid + i * NT;
        if (row < mrows) *reinterpret_cast<uint4*>(lds + row * D::XROW + kc * 16) = xv[row][i];
      }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

    // This wave's groups: P and X of each into LDS. The x operands of a
    // block are read while the previous block computes; when all of the
    // wave's blocks lie inside K (FULL) the blocks run without bound tests.
    // Lane groups g < GR store P (rows 4 g .. 4 g + 3 of their column, those
    // below MR), their lane 0 stores X; every other lane stores into its own 4
    // bytes of the dummy area. (The masks pass through an empty asm statement
    // so that each store address is computed where it is used.)
    const int64_t q0 = k0 >> 5;              // the round's first chunk-step
    const int64_t qw = q0 + 4 * wave * BPW;  // this wave's first chunk-step
    const bool prow = g < D::GR, xrow = prow && r16 == 0;
    uint32_t p_at = prow ? (uint32_t)(D::OFF_P + g * 256 + r16 * 4) : (uint32_t)(D::OFF_DUMMY + lane * 4);
    uint32_t p_gmask = prow ? ~0u : 0u;
    uint32_t x_at = xrow ? (uint32_t)(D::OFF_X + g * 16) : (uint32_t)(D::OFF_DUMMY + lane * 4);
    uint32_t x_gmask = xrow ? ~0u : 0u;
    asm volatile("" : "+v"(p_gmask), "+v"(x_gmask), "+v"(p_at), "+v"(x_at));
    const auto blocks = [&](auto full_tag) {
      constexpr bool FULL = decltype(full_tag)::value;
      uint4 av[2][4];
      const auto read_x = [&](int j, uint4 (&dst)[4]) {
#pragma unroll
        for (int jj = 0; jj < 4; jj++)
          dst[jj] = *reinterpret_cast<const uint4*>(lds + a_base + 64 * (uint32_t)(qw + 4 * j + jj - q0));
      };
      read_x(0, av[0]);
#pragma unroll
      for (int j = 0; j < BPW; j++) {
        const int64_t qb = qw + 4 * j;
        if (!FULL && qb >= nq) break;
        if (j + 1 < BPW) read_x(j + 1, av[(j + 1) & 1]);
        // After the transposes word set u of lane group g holds, at position
        // jj, its words of chunk-step 4 b + jj (4-bit: one word; 8-bit: the
        // even set the first, the odd set the second).
        uint32_t wu[WPL][4];
        if constexpr (QB == 2) {
          // Lane group i's 16 bits of chunk-step 4 b + g are half i % 2 of
          // word i / 2: widened to a word each before the transpose.
#pragma unroll
          for (int i = 0; i < 4; i++) wu[0][i] = (cw[j][i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
          xpose_lane_groups(wu[0]);
        } else {
#pragma unroll
          for (int u = 0; u < WPL; u++) {
#pragma unroll
            for (int i = 0; i < 4; i++) wu[u][i] = cw[j][WPL * i + u];
            xpose_lane_groups(wu[u]);
          }
        }
        f32x4_t P = zero, X = zero;
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
          const int64_t q = qb + jj;
          if (!FULL && q >= nq) break;
          uint4 bv;
          if constexpr (QB == 2)
            bv = codes2_as_elems<T>(wu[0][jj]);
          else if constexpr (QB == 4)
            bv = codes_as_elems<T>(wu[0][jj]);
          else
            bv = bytes_as_elems<T>(wu[0][jj], wu[1][jj]);
          const bool first = (jj % CPG) == 0;  // blocks start on group boundaries
          P = chunk_step(T(0), av[j & 1][jj], bv, first ? zero : P);
          X = chunk_step(T(0), av[j & 1][jj], ones, first ? zero : X);
          if ((jj % CPG) == CPG - 1) {
            const uint32_t gi = (uint32_t)((q - q0) / CPG);
#pragma unroll
            for (int e = 0; e < (MR < 4 ? MR : 4); e++) {
              *reinterpret_cast<float*>(lds + p_at + ((gi * (MR * 64) + e * 64) & p_gmask)) = P[e];
              *reinterpret_cast<float*>(lds + x_at + ((gi * D::XS + e * 4) & x_gmask)) = X[e];
            }
          }
        }
        // Keeps the scheduler from hoisting later blocks' operand reads.
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    if (qw + 4 * BPW <= nq)
      blocks(std::true_type{});
    else
      blocks(std::false_type{});
    float* ss = reinterpret_cast<float*>(lds + D::OFF_S);
    float* zs = reinterpret_cast<float*>(lds + D::OFF_Z);
#pragma unroll
    for (int i = 0; i < D::SPL; i++) {
      const int e = tid + i * NT, col = e / RG, gi = e % RG;
      ss[col * D::SRS + gi] = Elem<T>::to_f32(__builtin_bit_cast(T, sv[i]));
      zs[col * D::SRS + gi] = Elem<T>::to_f32(__builtin_bit_cast(T, zv[i]));
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

    if (wave < D::GR) {
      // The round's groups in ascending order, FC at a time, the operands of
      // the next FC read while these fold; wave w folds rows 4 w .. 4 w + 3.
      constexpr int FC = 8;
      const int e = 4 * wave + (lane >> 4), n = lane & 15;
      const int ng = (int)min((int64_t)RG, G - r * RG);
      uint32_t op = D::OFF_P + (e * 16 + n) * 4, ox = D::OFF_X + e * 4, os = n * D::SRS * 4;
      asm volatile("" : "+v"(op), "+v"(ox), "+v"(os));
      const float* Pf = reinterpret_cast<const float*>(lds + op);  // group gi: [MR * 16 gi]
      const float* Xf = reinterpret_cast<const float*>(lds + ox);  // [XS / 4 gi]
      const f32x4_t* Sf = reinterpret_cast<const f32x4_t*>(lds + D::OFF_S + os);
      const f32x4_t* Zf = reinterpret_cast<const f32x4_t*>(lds + D::OFF_Z + os);
      struct Ops {
        float p[FC], x[FC];
        f32x4_t s[FC / 4], z[FC / 4];
      };
      const auto load = [&](int c, Ops& o) {
#pragma unroll
        for (int i = 0; i < FC; i++) {
          o.p[i] = Pf[(c * FC + i) * MR * 16];
          o.x[i] = Xf[(c * FC + i) * (D::XS / 4)];
        }
#pragma unroll
        for (int i = 0; i < FC / 4; i++) {
          o.s[i] = Sf[c * (FC / 4) + i];
          o.z[i] = Zf[c * (FC / 4) + i];
        }
      };
      const auto fold = [&](const Ops& o) {
#pragma unroll
        for (int i = 0; i < FC; i++) {
          acc = __builtin_fmaf(o.s[i / 4][i % 4], o.p[i], acc);
          acc = __builtin_fmaf(o.z[i / 4][i % 4], o.x[i], acc);
        }
      };
      const int nfull = ng / FC;
      Ops o0, o1;
      if (nfull > 0) load(0, o0);
      for (int c = 0; c < nfull; c += 2) {
        if (c + 1 < nfull) load(c + 1, o1);
        fold(o0);
        if (c + 1 < nfull) {
          if (c + 2 < nfull) load(c + 2, o0);
          fold(o1);
        }
      }
      const float* Ss = reinterpret_cast<const float*>(Sf);
      const float* Zs = reinterpret_cast<const float*>(Zf);
      for (int gi = nfull * FC; gi < ng; gi++) {
        acc = __builtin_fmaf(Ss[gi], Pf[gi * MR * 16], acc);
        acc = __builtin_fmaf(Zs[gi], Xf[gi * (D::XS / 4)], acc);
      }
    }
    if (rr + 1 < rounds) asm volatile("s_barrier" ::: "memory");
  }

  if (wave < D::GR) {
    const int e = 4 * wave + (lane >> 4), n = lane & 15;
    if (e < mrows && n < cols) static_cast<T*>(p.out)[e * N + n0 + n] = Elem<T>::from_f32(acc);
  }
}

}  // namespace bi_gemm_dev
