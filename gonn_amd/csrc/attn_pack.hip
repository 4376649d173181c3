// attn_pack.hip -- fp32/bf16 (BH,S,D) rows -> the bf16 operand layouts the
// MFMA kernels read.
//
// Two layouts per source tensor X (BH,S,D), S padded to Sp (a multiple of 64,
// pad rows zero):
//   row  Xb (BH,Sp,D) bf16, row-major: an MFMA operand whose lanes each take
//        one row of X and 8 consecutive elements along D.
//   tr   Xt (BH,D,Sp) bf16, transposed, with the positions inside every group
//        of 16 permuted by vt_pos: an MFMA operand that contracts over the
//        sequence axis against P, dS (or their transposes) taken straight from
//        an accumulator, so each lane's 8 k-values are one 16-byte read.
// One launch packs up to two sources; either output of a source may be null.
#include "common.h"
#include "kernels.h"

namespace gonn {

template <typename T, int D>
GONN_DEV void load8(const T* p, float* v) {
    if constexpr (sizeof(T) == 4) {
        const f32x4 a = *(const f32x4*)p, b = *(const f32x4*)(p + 4);
        for (int i = 0; i < 4; i++) {
            v[i] = a[i];
            v[4 + i] = b[i];
        }
    } else {
        const u16x8 a = *(const u16x8*)p;
        for (int i = 0; i < 8; i++) v[i] = bf16_to_f32(a[i]);
    }
}

// grid (Sp/64, BH, nsrc), 256 threads.
template <typename T, int D>
__global__ __launch_bounds__(256) void pack_kernel(PackParams p) {
    constexpr int BN = 64;
    constexpr int VS = D + 2;
    __shared__ bf16 tile[BN * VS];
    const int tid = threadIdx.x;
    const int kt = blockIdx.x, bh = blockIdx.y, which = blockIdx.z;
    const T* src = (const T*)p.src[which];
    bf16* row = (bf16*)p.row[which];
    bf16* tr = (bf16*)p.tr[which];
    const int S = p.S, Sp = p.Sp;
    const size_t src0 = (size_t)bh * S * D;
    constexpr int CH = BN * D / 8;
    for (int c = tid; c < CH; c += 256) {
        const int r = c / (D / 8), col = (c % (D / 8)) * 8;
        const int key = kt * BN + r;
        float v[8];
        if (key < S) {
            load8<T, D>(src + src0 + (size_t)key * D + col, v);
        } else {
            for (int i = 0; i < 8; i++) v[i] = 0.f;
        }
        if (row)
            *(bf16x8*)(row + ((size_t)bh * Sp + key) * D + col) =
                pack8(v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]);
        if (tr)
            for (int i = 0; i < 8; i++) tile[r * VS + col + i] = to_bf16(v[i]);
    }
    if (!tr) return;  // uniform for the workgroup
    __syncthreads();
    constexpr int VC = D * BN / 8;
    for (int c = tid; c < VC; c += 256) {
        const int d = c / (BN / 8), j = c % (BN / 8);
        const int grp = (j >> 1) * 16;
        bf16x8 r;
        for (int i = 0; i < 8; i++) {
            const int pos = (j & 1) * 8 + i;
            r[i] = tile[(grp + vt_pos(pos)) * VS + d];
        }
        *(bf16x8*)(tr + ((size_t)bh * D + d) * Sp + kt * BN + j * 8) = r;
    }
}

hipError_t launch_pack(const PackParams& p, int nsrc, int in_bf16, int BH, int D, hipStream_t s) {
    if (nsrc < 1 || nsrc > 2 || p.Sp % 64 != 0) return hipErrorInvalidValue;
    dim3 grid(p.Sp / 64, BH, nsrc);
    if (D == 64) {
        if (in_bf16) pack_kernel<bf16, 64><<<grid, 256, 0, s>>>(p);
        else pack_kernel<float, 64><<<grid, 256, 0, s>>>(p);
    } else if (D == 128) {
        if (in_bf16) pack_kernel<bf16, 128><<<grid, 256, 0, s>>>(p);
        else pack_kernel<float, 128><<<grid, 256, 0, s>>>(p);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace gonn
