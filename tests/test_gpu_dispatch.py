"""Automatic kernel choice (no override) at the boundaries of its rules:
stream vs MFMA (M <= 16; M <= 64 unless K > 1024 with over 1024 stream
tiles; M <= 128 with at most 512 stream tiles), the LDS kernel's K >= 2048 gate and its
full-round rule below it (256 tiles of 256 x 64 vs 2.25 rounds), ragged N
and K, K that the LDS kernel cannot take (K % 256 != 0), and the MFMA
kernel's tile height (32, 48 or 64 rows, fewest rows per CU), and the K
split over workgroups for few tiles and long K (and none where it loses:
the BASELINE shapes).  Every output must equal the exact product, on two
calls in a row (the split's arrival counters return to zero)."""
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"
DENSE4 = (255, 253, 251, 247)

SHAPES = [
    (128, 768, 2304),    # MFMA 32 x 48 tiles: 576 stream tiles of 32 x 16 would be too many
    (256, 768, 1536),    # MFMA 32 x 48 tiles (256 of them)
    (256, 768, 3072),    # MFMA 64 x 48 tiles
    (250, 1024, 3070),   # MFMA 64 x 48 tiles, ragged M and N
    (96, 768, 2304),     # stream: 432 tiles
    (128, 768, 768),     # stream: 192 tiles
    (64, 768, 4608),     # stream (M <= 64, K <= 1024)
    (16, 2048, 12288),   # stream (M <= 16)
    (32, 2048, 8192),    # stream: K > 1024 but 1024 stream tiles of 16 x 16
    (24, 2048, 12288),   # MFMA 32-row tiles (K > 1024, 1536 stream tiles)
    (40, 2048, 12288),   # MFMA 48-row tiles
    (64, 2048, 12288),   # MFMA 64-row tiles
    (128, 4096, 4096),   # MFMA past K = 1024: 64-row tiles
    (129, 768, 2304),    # MFMA (M > 128)
    (64, 4096, 1000),    # stream, ragged N
    (512, 4096, 12288),  # LDS, K >= 2048
    (1024, 2048, 4096),  # LDS at the K gate, 256 tiles
    (512, 2048, 4096),   # MFMA: 128 LDS tiles are too few
    (1024, 1024, 4096),  # LDS below the K gate: 256 tiles, one full round
    (4096, 768, 2304),   # MFMA: 576 LDS tiles would be 2.25 rounds
    (1024, 1024, 4090),  # LDS with ragged N (columns clamped)
    (1000, 1088, 4096),  # K % 256 != 0: MFMA
    (300, 100, 37),      # ragged everything: K padded to 128
    (224, 768, 2304),    # MFMA 32 x 64 tiles: 252 fit one round
    (256, 768, 2304),    # MFMA 48 x 64 tiles: 216 in one round (the headline shape)
    (250, 768, 2290),    # 48 x 64 tiles with ragged M and N
    (384, 768, 2304),    # MFMA 64 x 64 tiles: 216 (48 rows would need 288)
    (256, 768, 4608),    # no height fits one round: 48 rows (2 rounds) ties 32 (3)
    (4096, 768, 768),    # C4 out_proj: MFMA 64 x 64 tiles
    # K split over workgroups
    (1, 16384, 768),     # decode: 8 one-wave splits
    (3, 4096, 770),      # decode: 4 splits, ragged N
    (1, 2048, 768),      # 2 splits would be the cap: 4 waves in one workgroup instead
    (256, 8192, 256),    # MFMA 32 x 64, 8 splits
    (250, 4096, 760),    # MFMA, 4 splits, ragged M and N
    (512, 8192, 512),    # 128 tiles, K >= 8192: 2 splits
    (2048, 16384, 768),  # 384 tiles of 64 x 64, 2 splits
]


@pytest.mark.parametrize("m,k,n", SHAPES)
def test_auto_choice_is_exact(backend, m, k, n):
    gen = torch.Generator(device=DEV).manual_seed(m * 7 + k + n)
    w = torch.randint(-127, 128, (n, k), generator=gen, device=DEV, dtype=torch.int8)
    a = torch.randint(-127, 128, (m, k), generator=gen, device=DEV, dtype=torch.int8)
    prepared = backend.prepare_weight_nk(w, DENSE4)
    ws = backend.create_workspace(device=torch.device(DEV), channels=4, m=m, n=n, k=k)
    want = a.double() @ w.double().t()  # exact: integer sums below 2^53
    for _ in range(2):
        out = backend.matmul_prepared_fused(a, prepared, workspace=ws)
        assert torch.equal(out.double(), want)
