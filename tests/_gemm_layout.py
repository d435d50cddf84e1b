"""The Q4_0 GEMM tile layout of include/miattn.h (mia_q4_0_pack_gemm), restated
with numpy index arithmetic, and the kernel's operand formation from it
(q4_gemm_wide_kernel, tile layout) emulated on the CPU."""

import numpy as np

ORDER = np.array([0, 2, 1, 3, 4, 6, 5, 7])


def pack_layout(W, N, K):
    """Tile (s, i) at (s * K / 64 + i) * 2304: quant bytes at h * 1024 + row *
    16 + 8 * block + j (byte 8 h + ORDER[j] of the block's 16), then the fp16
    scales at 2048 + row * 4 + 2 * block.  W: [N][K / 32 * 18] bytes (or any
    array of that many items, to follow where each item goes)."""
    rows = W.reshape(N // 64, 64, K // 64, 36)               # [slab][row][step][2 blocks]
    out = np.zeros((N // 64, K // 64, 2304), W.dtype)
    rr = np.arange(64)
    for bb in range(2):
        for e in range(2):                                    # the fp16 scale's two bytes
            out[:, :, 2048 + rr * 4 + 2 * bb + e] = rows[:, :, :, 18 * bb + e].transpose(0, 2, 1)
        for h in range(2):
            for j in range(8):
                src = 18 * bb + 2 + 8 * h + ORDER[j]
                out[:, :, h * 1024 + rr * 16 + 8 * bb + j] = rows[:, :, :, src].transpose(0, 2, 1)
    return out.reshape(-1)


def dequant_from_layout(P, N, K):
    """The weights as the kernel forms them from a packed matrix: lane (row,
    half h) reads its 16 quant bytes and the row's scale pair; the B operand
    dword t of k-step ks in block bb is ((dword >> (8 (t & 1) + 4 ks)) &
    0x000F000F) - 8 per half, holding values 16 ks + 8 h + 2 t, + 1."""
    steps = K // 64
    out = np.zeros((N, K))
    tiles = P.reshape(N // 64, steps, 2304)
    for n in range(N):
        s, rr = divmod(n, 64)
        for i in range(steps):
            tile = tiles[s, i]
            sc = tile[2048 + rr * 4:2048 + rr * 4 + 4].view(np.float16).astype(np.float64)
            for h in range(2):
                q = tile[h * 1024 + rr * 16:h * 1024 + rr * 16 + 16].view(np.uint32)
                for bb in range(2):
                    for ks in range(2):
                        for t in range(4):
                            x = int(q[2 * bb + (t >> 1)]) >> (8 * (t & 1) + 4 * ks)
                            k0 = 64 * i + 32 * bb + 16 * ks + 8 * h + 2 * t
                            out[n, k0] = ((x & 0xF) - 8) * sc[bb]
                            out[n, k0 + 1] = (((x >> 16) & 0xF) - 8) * sc[bb]
    return out
