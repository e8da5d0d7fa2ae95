// Tiled fp16 GEMM on the gfx950 matrix cores for the encoder-sized products (M = clips x 1500 or x 3000):
// QKV (head-major scatter), out-proj and fc2 (residual add into the fp32 stream), fc1 (GELU), the conv stem as an
// implicit GEMM (no im2col buffer), and the cross-attention K/V of every decoder layer. Replaces the reference's
// cuBLAS calls with a bias prefill (src/gpu.rs:208-236, 254-286; kernels/whisper.cu:92-104, 106-139).
//
// Block tile BM x BN x 64 with 8 waves in a 2 x 4 grid (two waves per SIMD, so one wave's LDS reads overlap the
// other's products); each wave owns a (BM/2) x (BN/4) tile of 32x32x16 MFMA products. Both operands are
// K-contiguous and go from global memory straight into LDS (buffer_load ... lds, 16 bytes per lane, no register
// staging), double buffered: the loads of K tile k + 1 are in flight while tile k is multiplied, with one barrier per
// K tile; the operand fragments are software pipelined a 16-wide K step ahead of the products. In LDS a tile row is 64 halves (128 bytes) whose 16-byte chunks are XOR-swizzled by the row index (chunk c
// of row r sits at position c ^ (r % 8) ^ (r / 8 % 2)): the 16 lanes that one ds_read_b128 cycle serves read 16
// consecutive rows at one chunk, and these land in 16 distinct 16-byte bank groups of the 256-byte bank row; a
// direct load writes lane i's 16 bytes at base + 16 i, so each lane fetches the global chunk that belongs at its
// swizzled position. Rows past the end of an operand (and the zero padding of the implicit convolution) are read
// through the buffer descriptor's range check, which returns zeros.
// The activation tile is the MFMA A operand and the W tile the B operand, so lane l of a 32x32 product holds output
// column l % 32 of eight rows: every store instruction writes two 32-column row segments. The transposed tiles of
// the encoder's v are staged through LDS to be written as runs of token positions.
#include "mz_common.h"
#include "mz_kernels.h"

namespace {

constexpr int NW = 8;  // waves per workgroup
typedef __attribute__((address_space(3))) void lds_void;
#define LDSP(p) ((lds_void*)(p))
constexpr unsigned OOB = 0x80000000u;  // a buffer offset past every operand: the load returns zeros

// Workgroup i runs on XCD i % 8, and each XCD has its own L2. XCD x owns a band of rows = ceil(nbm / 8) block rows
// and visits its tiles with the block row fastest: the band's activation panels stay in its L2 while each weight
// panel is read once per XCD and shared by the band's tiles that run at the same time. The grid is 8 * rows * nbn.
__device__ __forceinline__ bool xcd_tile(int bid, int nbm, int nbn, int* bm, int* bn) {
    const int rows = (nbm + 7) >> 3, li = bid >> 3;
    *bm = (bid & 7) * rows + li % rows;
    *bn = li / rows;
    return *bm < nbm && *bn < nbn;
}

template <int BM, int BN, int ALOAD, int EPI>
__global__ void __launch_bounds__(NW * 64) gemm_kernel(const MzGemm p) {
#if defined(__HIP_DEVICE_COMPILE__)  // the buffer-resource type exists only in the device pass
    constexpr int WM = BM / 2, WN = BN / 4, TM = WM / 32, TN = WN / 32;
    constexpr int AR = BM / (8 * NW), WR = BN / (8 * NW);  // 8-row slices each wave loads per K tile
    static_assert(AR >= 1 && WR >= 1 && TN >= 1, "tile too small for 8 waves");
    __shared__ __attribute__((aligned(16))) f16 sA0[BM * 64];
    __shared__ __attribute__((aligned(16))) f16 sA1[BM * 64];
    __shared__ __attribute__((aligned(16))) f16 sW0[BN * 64];
    __shared__ __attribute__((aligned(16))) f16 sW1[BN * 64];

    const int nbn = (p.N + BN - 1) / BN, nbm = (p.M + BM - 1) / BM;
    // Plain products run a persistent grid (one workgroup per CU) over xcd_tile's virtual tile order: workgroup w
    // takes virtual tiles w, w + G, w + 2 G, ... (G a multiple of 8, so all of a workgroup's tiles lie on its XCD),
    // and the next tile's first K tile is requested before this tile's epilogue runs, so its round trip and the
    // workgroup's dispatch are not paid once per tile. The convolution takes one tile per workgroup.
    constexpr bool PERSIST = ALOAD == ALOAD_PLAIN;
    const int nvirt = 8 * ((nbm + 7) >> 3) * nbn, vstep = PERSIST ? (int)gridDim.x : nvirt;
    int v = blockIdx.x, bm = 0, bn = 0;
    while (v < nvirt && !xcd_tile(v, nbm, nbn, &bm, &bn)) v += vstep;
    if (v >= nvirt) return;
    // the wave index through readfirstlane: wave-uniform values (tile origins, store descriptors) stay scalar
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 2, wn = wave & 3, lr = lane & 31, lh = lane >> 5;
    // the epilogue's bias values are requested here, ahead of the operand loads, so that their round trip is hidden
    // behind the K loop instead of stalling the products' end. One unconditional buffer load per column block (a
    // missing bias is a descriptor of no bytes, which reads zeros): a branch would make the compiler wait for the
    // load at once. Kept as fp16 until used.
    int n0 = bn * BN + wn * WN;
    const __amdgpu_buffer_rsrc_t rB = rsrc(p.bias, p.bias ? (unsigned)p.N * 2 : 0u);
    f16 bias_h[TN];
#pragma unroll
    for (int j = 0; j < TN; j++)
        bias_h[j] = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(rB, (unsigned)(n0 + j * 32 + lr) * 2, 0, 0));
    const int nk = p.K >> 6;
    // this lane's slot in a direct load: row lrow of an 8-row slice, 16-byte chunk lc of the row
    // (slice r of a wave starts at a multiple of 8 rows whose bit 3 is r's bit 0)
    const int lrow = lane >> 3, lc = (lane & 7) ^ lrow;
    static_assert((BM / NW) % 16 == 0 && (BN / NW) % 16 == 0, "a wave's slices must start on a 16-row boundary");

    const __amdgpu_buffer_rsrc_t rW = rsrc(p.W, (unsigned)p.N * p.K * 2);
    unsigned voW[WR];
    auto set_w = [&](int bn_) {
#pragma unroll
        for (int r = 0; r < WR; r++)
            voW[r] = (unsigned)(bn_ * BN + wave * (BN / NW) + 8 * r + lrow) * p.K * 2 + (lc ^ (r & 1)) * 16;
    };
    set_w(bn);
    __amdgpu_buffer_rsrc_t rA;
    unsigned voA[AR];
    int srow[AR], stime[AR];  // conv: source row of tap 0 and its time index (-1 .. tin - 1), or a row past M
    auto set_a = [&](int bm_) {
#pragma unroll
        for (int r = 0; r < AR; r++)
            voA[r] = (unsigned)(bm_ * BM + wave * (BM / NW) + 8 * r + lrow) * p.lda * 2 + (lc ^ (r & 1)) * 16;
    };
    if (ALOAD == ALOAD_PLAIN) {
        rA = rsrc(p.A, (unsigned)p.M * p.lda * 2);
        set_a(bm);
    } else {
        const int clips = p.M / p.conv_tout;
        rA = rsrc(p.A, (unsigned)clips * p.conv_tin * p.conv_cin * 2);
#pragma unroll
        for (int r = 0; r < AR; r++) {
            const int m = bm * BM + wave * (BM / NW) + 8 * r + lrow;
            const int g = m / p.conv_tout, t = m - g * p.conv_tout;
            stime[r] = m < p.M ? p.conv_stride * t - 1 : -(1 << 20);
            srow[r] = g * p.conv_tin + p.conv_stride * t - 1;
        }
    }

    auto issue = [&](int kt, f16* a, f16* w) {
        if (ALOAD == ALOAD_PLAIN) {
#pragma unroll
            for (int r = 0; r < AR; r++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, LDSP(a + (wave * (BM / NW) + 8 * r) * 64), 16, voA[r],
                                                         kt * 128, 0, 0);
        } else {
            // implicit im2col: column k = tap * cin + ci of a row reads source time stride * t + tap - 1
            int tap2[2], ci2[2];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int k0 = kt * 64 + (lc ^ h) * 8;
                tap2[h] = k0 / p.conv_cin;
                ci2[h] = k0 - tap2[h] * p.conv_cin;
            }
#pragma unroll
            for (int r = 0; r < AR; r++) {
                const int tap = tap2[r & 1], ci = ci2[r & 1];
                const int tt = stime[r] + tap;
                const bool ok = tap < 3 && tt >= 0 && tt < p.conv_tin;
                const unsigned vo = ok ? (unsigned)((srow[r] + tap) * p.conv_cin + ci) * 2 : OOB;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, LDSP(a + (wave * (BM / NW) + 8 * r) * 64), 16, vo, 0, 0,
                                                         0);
            }
        }
#pragma unroll
        for (int r = 0; r < WR; r++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rW, LDSP(w + (wave * (BN / NW) + 8 * r) * 64), 16, voW[r],
                                                     kt * 128, 0, 0);
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = f32x16{};
    // Fragments of K step kk (16 wide) of a tile: TM A and TN W fragments. They are double buffered across steps:
    // step kk + 1's reads go out while step kk's products issue, one read between two products (explicit scheduling
    // groups; the hardware interleaves the two waves of a SIMD on top). The last step's products are split around
    // the tile's wait and barrier, so that the next tile's first fragments are read under the second half.
    f16x8 fa0[TM], fw0[TN], fa1[TM], fw1[TN];
    auto frags = [&](const f16* a, const f16* w, int kk, f16x8(&fa)[TM], f16x8(&fw)[TN]) {
        const int sw = (((2 * kk + lh) ^ (lr & 7) ^ ((lr >> 3) & 1)) << 3);
#pragma unroll
        for (int i = 0; i < TM; i++) fa[i] = *(const f16x8*)&a[(wm * WM + i * 32 + lr) * 64 + sw];
#pragma unroll
        for (int j = 0; j < TN; j++) fw[j] = *(const f16x8*)&w[(wn * WN + j * 32 + lr) * 64 + sw];
    };
    auto mma = [&](const f16x8(&fa)[TM], const f16x8(&fw)[TN], int i0, int i1) {
#pragma unroll
        for (int i = i0; i < i1; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) acc[i][j] = mfma32(fa[i], fw[j], acc[i][j]);
    };
    constexpr int NM = TM * TN, NR = TM + TN, NI = NM < NR ? NM : NR;  // products, reads, interleaved pairs
    auto interleave = [&]() {
#pragma unroll
        for (int g = 0; g < NI; g++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
        }
        if (NM > NI) __builtin_amdgcn_sched_group_barrier(0x008, NM - NI, 0);
        if (NR > NI) __builtin_amdgcn_sched_group_barrier(0x100, NR - NI, 0);
    };
    // tile kt from (a, w), its step-0 fragments already in (fa0, fw0); the loads of tile kt + 1 go to (an, wn_)
    auto tile = [&](int kt, const f16* a, const f16* w, f16* an, f16* wn_) {
        if (kt + 1 < nk) issue(kt + 1, an, wn_);
        frags(a, w, 1, fa1, fw1);
        mma(fa0, fw0, 0, TM);
        __builtin_amdgcn_sched_group_barrier(0x020, AR + WR, 0);  // the next tile's loads first
        interleave();
        frags(a, w, 2, fa0, fw0);
        mma(fa1, fw1, 0, TM);
        interleave();
        frags(a, w, 3, fa1, fw1);
        mma(fa0, fw0, 0, TM);
        interleave();
        mma(fa1, fw1, 0, TM / 2);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(0);  // tile kt + 1 has landed (vmcnt) and every wave is done with tile kt
        __syncthreads();
        if (kt + 1 < nk) frags(an, wn_, 0, fa0, fw0);
        mma(fa1, fw1, TM / 2, TM);
        __builtin_amdgcn_sched_barrier(0);
    };

    // epilogue: acc[i][j] element r is row m0 + i * 32 + 8 (r / 4) + 4 lh + r % 4, column n0 + j * 32 + lr
    auto epilogue = [&](const int m0, const int n0) {
    if (EPI == EPI_HEADS) {
        if (p.kind == 3) lds_barrier();  // every wave is done reading operands: LDS is free for the v transposes
        const int blk = n0 >> 6;           // a wave's columns lie in one 64-wide head block (WN <= 64)
        const bool vt = p.kind == 3 && blk / p.nh == 2;
        if (vt) {
            // encoder v: stage each 32-row slice of the wave's tile in LDS as [column][row] (the wave's own 32 x WN
            // halves of sW1, which the next tile's first loads leave alone: 8 waves x 32 x WN <= BN x 64) and write
            // runs of 4 token positions
            static_assert(NW * 32 * WN <= BN * 64, "staging slice exceeds sW1");
            f16* st = sW1 + wave * (32 * WN);
#pragma unroll
            for (int i = 0; i < TM; i++) {
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    const float bv = (float)bias_h[j];
#pragma unroll
                    for (int r = 0; r < 16; r++)
                        st[(j * 32 + lr) * 32 + 8 * (r >> 2) + 4 * lh + (r & 3)] = (f16)(acc[i][j][r] + bv);
                }
                __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the slice is in LDS (stores in flight stay)
                __builtin_amdgcn_wave_barrier();
#pragma unroll
                for (int c = lane; c < WN * 8; c += 64) {
                    const int nl = c >> 3, ml = (c & 7) * 4;
                    const int m = m0 + i * 32 + ml, n = n0 + nl;
                    if (m < p.M && n < p.N) {
                        const int g = m / MZ_TENC, t = m - g * MZ_TENC;  // 4 | 1500: the run stays in one clip
                        f16* dst = p.heads + ((long)(p.slot0 + g) * p.blocks_per_clip + (n >> 6)) * (MZ_TPAD * MZ_HD) +
                                   (long)(n & 63) * MZ_TPAD + t;
                        *(f16x4*)dst = *(const f16x4*)&st[nl * 32 + ml];
                    }
                }
                __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
                __builtin_amdgcn_wave_barrier();  // the slice is read before the next one overwrites it
            }
            return;
        }
    }
    // row offsets of accumulator element r within a 32-row product: 8 (r / 4) + r % 4 (+ 4 for the upper half-wave)
    if (EPI == EPI_HEADS) {
        // q and k tiles (and every tile of kind 2) are row-major [t][64]. M is a whole number of clips, and a
        // wave's 128 rows span at most two of them (128 < 1500): the store descriptor starts at the first one's
        // tiles and ends after the second one, or after the last clip of the call, so the range check drops the
        // rows of a partial last tile. Rows of the second clip add one clip's worth of tiles; every offset stays
        // below 2^31 bytes (two clips of at most 4096 tiles).
        const int g0 = m0 / MZ_TENC;
        const long clip = (long)p.blocks_per_clip * (MZ_TPAD * MZ_HD);
        const int ncl = min(p.M / MZ_TENC - g0, 2);
        const __amdgpu_buffer_rsrc_t rH =
            rsrc(p.heads + (p.slot0 + g0) * clip, ncl > 0 ? (unsigned)(ncl * clip * 2) : 0u);
        const int blk = n0 >> 6, c0 = (n0 & 63) + lr;
        // the encoder's q tiles are stored multiplied by log2(e) / 8, the attention's exponent scale
        const float qsc = (p.kind == 3 && blk < p.nh) ? 0.125f * 1.4426950408889634f : 1.f;
        float bv[TN];
#pragma unroll
        for (int j = 0; j < TN; j++) bv[j] = (float)bias_h[j] * qsc;
        // frame tb + dr >= 1500 is frame tb + dr - 1500 of the next clip
        const unsigned wrap = (unsigned)(clip - MZ_TENC * MZ_HD);
#pragma unroll
        for (int i = 0; i < TM; i++) {
            const int mb = m0 + i * 32 + 4 * lh, gb = mb / MZ_TENC, tb = mb - gb * MZ_TENC;
            const unsigned cb = (unsigned)((gb - g0) * clip + (long)blk * (MZ_TPAD * MZ_HD)) + c0 + tb * MZ_HD;
            if ((m0 + i * 32) / MZ_TENC == (m0 + i * 32 + 31) / MZ_TENC) {
                // the block's 32 rows lie in one clip (wave-uniform; all but one block in 47 at 1500 rows per clip):
                // each element's offset from cb is a constant, carried in the instruction's immediate offset
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int dr = 8 * (r >> 2) + (r & 3);
#pragma unroll
                    for (int j = 0; j < TN; j++)
                        __builtin_amdgcn_raw_buffer_store_b16(
                            __builtin_bit_cast(short, (f16)fmaf(acc[i][j][r], qsc, bv[j])), rH, cb * 2 + (dr * MZ_HD * 2 + j * 64),
                            0, 0);
                }
                continue;
            }
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int dr = 8 * (r >> 2) + (r & 3);
                const unsigned e = cb + dr * MZ_HD + (tb + dr >= MZ_TENC ? wrap : 0u);
                // a row's 32-column blocks back to back (the later ones through the immediate offset): the two halves
                // of a 128-byte tile row are written together
#pragma unroll
                for (int j = 0; j < TN; j++)
                    __builtin_amdgcn_raw_buffer_store_b16(
                        __builtin_bit_cast(short, (f16)fmaf(acc[i][j][r], qsc, bv[j])), rH, e * 2 + j * 64, 0, 0);
            }
        }
        return;
    }
    if (EPI == EPI_F16 || EPI == EPI_GELU_F16 || EPI == EPI_RESID_F32) {
        // buffer stores over exactly M rows: the range check drops the rows of a partial last tile, and every
        // offset is one lane base plus a wave-uniform row offset
        constexpr unsigned ES = EPI == EPI_RESID_F32 ? 4 : 2;
        const __amdgpu_buffer_rsrc_t rO = rsrc(p.out, (unsigned)(p.M * p.ldo) * ES);
        // the row stride as an opaque scalar: each element's offset is then one vector add of a scalar row offset
        const unsigned rs = __builtin_amdgcn_readfirstlane((unsigned)p.ldo * ES);
        auto put = [&](float v, unsigned o) {
            if (EPI == EPI_F16) {
                __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(short, (f16)v), rO, o, 0, 0);
            } else if (EPI == EPI_GELU_F16) {
                __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(short, (f16)gelu_erf_h(v)), rO, o, 0, 0);
            } else {
                const float x = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rO, o, 0, 0));
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, x + v), rO, o, 0, 0);
            }
        };
        // rows m0 + 4 lh + i * 32 + 8 (r / 4) + r % 4 in order: one row further, five after every fourth
        const unsigned off0 = (unsigned)((m0 + 4 * lh) * p.ldo + n0 + lr) * ES;
        if (n0 + WN <= p.N) {
            // every column of the wave exists (wave-uniform): the TN column blocks of a row are stored back to back,
            // the later ones through the instruction's immediate offset, so the two halves of a 128-byte line are
            // written together rather than 64 stores apart
            float bv[TN];
#pragma unroll
            for (int j = 0; j < TN; j++) bv[j] = (float)bias_h[j];
            unsigned off = off0;
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int r = 0; r < 16; r++, off += (r & 3) == 0 ? 5 * rs : rs)
#pragma unroll
                    for (int j = 0; j < TN; j++) put(acc[i][j][r] + bv[j], off + j * 32 * ES);
        } else {
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int n = n0 + j * 32 + lr;
                if (n >= p.N) continue;
                const float bv = (float)bias_h[j];
                unsigned off = off0 + j * 32 * ES;
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int r = 0; r < 16; r++, off += (r & 3) == 0 ? 5 * rs : rs) put(acc[i][j][r] + bv, off);
            }
        }
        return;
    }
    // EPI_GELU_POS (the conv stem's second product, once per encoder pass)
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int n = n0 + j * 32 + lr;
        if (n >= p.N) continue;
        const float bv = (float)bias_h[j];
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + i * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                if (m >= p.M) continue;
                const float v = acc[i][j][r] + bv;
                ((float*)p.out)[(long)m * p.ldo + n] = gelu_erf(v) + (float)p.pos[(long)(m % MZ_TENC) * p.N + n];
            }
    }
    };

    // two K tiles per iteration, one per LDS buffer (distinct arrays, so the compiler sees that the loads in flight
    // never alias the tile being read); an odd last tile is left in buffer 0. After the K loop every read of both
    // buffers is done (the last tile's barrier), so the next tile's first K tile can go to buffer 0 at once.
    issue(0, sA0, sW0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    frags(sA0, sW0, 0, fa0, fw0);
    for (;;) {
        int kt = 0;
        for (; kt + 1 < nk; kt += 2) {
            tile(kt, sA0, sW0, sA1, sW1);
            tile(kt + 1, sA1, sW1, sA0, sW0);
        }
        if (kt < nk) tile(kt, sA0, sW0, sA1, sW1);
        const int m0 = bm * BM + wm * WM, n0c = n0;
        int vn = v + vstep, bmn = 0, bnn = 0;
        while (vn < nvirt && !xcd_tile(vn, nbm, nbn, &bmn, &bnn)) vn += vstep;
        const bool more = PERSIST && vn < nvirt;
        f16 bias_n[TN];
        if (more) {  // the next tile's biases and first K tile, in flight during this epilogue
            // (the biases first: the compiler waits for their registers before the epilogue, and loads complete in
            // order, so the K tile issued after them stays in flight)
            n0 = bnn * BN + wn * WN;
#pragma unroll
            for (int j = 0; j < TN; j++)
                bias_n[j] = __builtin_bit_cast(
                    f16, __builtin_amdgcn_raw_buffer_load_b16(rB, (unsigned)(n0 + j * 32 + lr) * 2, 0, 0));
            set_a(bmn);
            set_w(bnn);
            issue(0, sA0, sW0);
        }
        epilogue(m0, n0c);
        if (!more) break;
        v = vn;
        bm = bmn;
        bn = bnn;
#pragma unroll
        for (int j = 0; j < TN; j++) bias_h[j] = bias_n[j];
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) acc[i][j] = f32x16{};
        __builtin_amdgcn_s_waitcnt(0);  // the next tile's first K tile has landed (and this tile's stores)
        __syncthreads();
        frags(sA0, sW0, 0, fa0, fw0);
    }
#endif
}

// compute units of the current device (workgroups of a persistent grid: one per CU), a multiple of 8
int cu_groups() {
    static int cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cached[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 8) n = 256;
        cached[dev] = n / 8 * 8;
    }
    return cached[dev];
}

template <int BM, int BN, int ALOAD, int EPI>
hipError_t launch(hipStream_t s, const MzGemm& g) {
    const int nbm = (g.M + BM - 1) / BM, nbn = (g.N + BN - 1) / BN;
    const int nvirt = 8 * ((nbm + 7) / 8) * nbn;
    const int cus = cu_groups(), grid = ALOAD == ALOAD_PLAIN && nvirt > cus ? cus : nvirt;
    hipLaunchKernelGGL((gemm_kernel<BM, BN, ALOAD, EPI>), dim3(grid), dim3(NW * 64), 0, s, g);
    return hipGetLastError();
}

template <int ALOAD, int EPI>
hipError_t pick(hipStream_t s, const MzGemm& g) {
    // 256 x 256 tiles once they cover most of the 256 CUs; 256 x 128, then 128 x 128 below that
    const long t256 = (long)((g.M + 255) / 256) * ((g.N + 255) / 256);
    if (t256 >= 200) return launch<256, 256, ALOAD, EPI>(s, g);
    const long t128 = (long)((g.M + 255) / 256) * ((g.N + 127) / 128);
    if (t128 >= 200) return launch<256, 128, ALOAD, EPI>(s, g);
    return launch<128, 128, ALOAD, EPI>(s, g);
}

}  // namespace

hipError_t mz_gemm_launch(hipStream_t s, int aload, int epi, const MzGemm& g) {
    if (g.K % 64 != 0 || g.M <= 0 || g.N <= 0 || g.K <= 0 || g.N % 4 != 0) return hipErrorInvalidValue;
    // (the head-scatter offsets span two clips of blocks_per_clip 1536 x 64 tiles: 4096 keeps them below 2^31 bytes;
    // large-v3's cross k/v is 32 layers x 2 x 20 heads = 1280 tiles per clip)
    if (epi == EPI_HEADS && (g.N % 64 != 0 || g.M % MZ_TENC != 0 || g.blocks_per_clip <= 0 || g.blocks_per_clip > 4096))
        return hipErrorInvalidValue;
    // the store descriptors address the output with 32-bit byte offsets
    if ((epi == EPI_F16 || epi == EPI_GELU_F16 || epi == EPI_RESID_F32) &&
        (long)g.M * g.ldo * (epi == EPI_RESID_F32 ? 4 : 2) >= (1L << 31))
        return hipErrorInvalidValue;
    if (aload == ALOAD_CONV) {
        if (g.conv_cin % 8 != 0 || g.conv_tout <= 0) return hipErrorInvalidValue;
        if (epi == EPI_GELU_F16) return pick<ALOAD_CONV, EPI_GELU_F16>(s, g);
        if (epi == EPI_GELU_POS) return pick<ALOAD_CONV, EPI_GELU_POS>(s, g);
        return hipErrorInvalidValue;
    }
    switch (epi) {
        case EPI_F16: return pick<ALOAD_PLAIN, EPI_F16>(s, g);
        case EPI_GELU_F16: return pick<ALOAD_PLAIN, EPI_GELU_F16>(s, g);
        case EPI_RESID_F32: return pick<ALOAD_PLAIN, EPI_RESID_F32>(s, g);
        case EPI_HEADS: return pick<ALOAD_PLAIN, EPI_HEADS>(s, g);
    }
    return hipErrorInvalidValue;
}
