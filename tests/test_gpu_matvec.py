"""GPU parity of lmx_matvec against the oracle's `dot_row` restatement
(crates/gguf/src/quant.rs:187-271) for every block format the path takes.

Tolerance: max|y - ref| <= 3e-5 * max|ref|: both sum thousands of f32
products, in different orders (the oracle per 32-element sub-block as the
reference does, the GPU per lane then across lanes)."""
import sys

import numpy as np
import pytest

import oracle

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import llmoxide_amd as lmx  # noqa: E402

TYPES = ["q4_k", "q6_k", "q8_0", "f32", "f16", "bf16"]


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def run(name, rows, in_dim, n_tok, seed):
    say(f"matvec {name} rows={rows} in_dim={in_dim} n_tok={n_tok}")
    ty = oracle.QTYPES[name]
    w = oracle.quant_weights(ty, rows, in_dim, seed)
    x = oracle.normal(seed + 50, (n_tok, in_dim))
    ref = oracle.matvec(ty, w, rows, in_dim, x)
    y = lmx.matvec(torch.from_numpy(w).cuda(), torch.from_numpy(x).cuda(), qtype=name, rows=rows,
                   in_dim=in_dim)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    err = np.abs(got - ref).max()
    assert err <= 3e-5 * np.abs(ref).max(), f"{name}: max err {err} vs max |ref| {np.abs(ref).max()}"


@pytest.mark.parametrize("name", TYPES)
def test_attn_output_shape_decode(name):
    # Qwen3-8B attn_output: 4096 x 4096, one token
    run(name, 4096, 4096, 1, seed=1)


@pytest.mark.parametrize("name", TYPES)
@pytest.mark.parametrize("n_tok", [2, 4, 7])
def test_ragged_rows_and_token_tiles(name, n_tok):
    # rows not a multiple of the 16 a workgroup takes; 7 tokens = two launches
    run(name, 37, 512, n_tok, seed=2 + n_tok)


@pytest.mark.parametrize("name", ["q4_k", "q6_k", "q8_0"])
def test_widest_rows(name):
    run(name, 64, 16384, 1, seed=9)


def test_odd_q6k_block_count_per_row():
    # 3 blocks per row: half the blocks start 2 bytes past a dword boundary
    run("q6_k", 33, 768, 2, seed=10)


@pytest.mark.parametrize("name", ["q4_k", "q6_k", "q8_0"])
@pytest.mark.parametrize("rows,in_dim,n_tok", [(70, 2560, 1), (41, 6400, 1), (41, 12544, 3)])
def test_partial_and_multiple_chunks(name, rows, in_dim, n_tok):
    # Q6_K and Q8_0 rows staged through LDS in 64-unit chunks: 40 units (one
    # partial chunk), 100 units (a full and a partial one) and 196 units
    # (three full chunks and a 4-unit one); odd Q6_K blocks per row put the
    # chunks' windows at every 2-byte offset mod 16.
    run(name, rows, in_dim, n_tok, seed=11 + rows + n_tok)


# ---- the matrix-core GEMM (n_tok >= 16, Q4_K / Q6_K / Q8_0): same bar --
GEMM_TYPES = ["q4_k", "q6_k", "q8_0"]


def run_rows(name, rows, in_dim, n_tok, seed, check_rows):
    """GEMM over the whole matrix, oracle on the listed rows only."""
    say(f"gemm {name} rows={rows} in_dim={in_dim} n_tok={n_tok} checked rows={len(check_rows)}")
    ty = oracle.QTYPES[name]
    w = oracle.quant_weights(ty, rows, in_dim, seed)
    x = oracle.normal(seed + 50, (n_tok, in_dim))
    y = lmx.matvec(torch.from_numpy(w).cuda(), torch.from_numpy(x).cuda(), qtype=name, rows=rows,
                   in_dim=in_dim)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    rb = oracle.row_bytes(ty, in_dim)
    sub = np.ascontiguousarray(w.reshape(rows, rb)[check_rows])
    ref = oracle.matvec(ty, sub, len(check_rows), in_dim, x)
    err = np.abs(got[:, check_rows] - ref).max()
    assert err <= 3e-5 * np.abs(ref).max(), f"{name}: max err {err} vs max |ref| {np.abs(ref).max()}"
    assert np.all(np.isfinite(got))


@pytest.mark.parametrize("name", GEMM_TYPES)
@pytest.mark.parametrize("n_tok", [16, 64])
def test_gemm_attn_output_shape(name, n_tok):
    # Qwen3-8B attn_output 4096 x 4096 at the GEMM threshold and one token block
    run(name, 4096, 4096, n_tok, seed=20 + n_tok)


@pytest.mark.parametrize("name", GEMM_TYPES)
def test_gemm_prefill_chunk_512(name):
    # the benched shape: a 512-token chunk through attn_output; every token,
    # rows from the first, a middle and the last row block
    rows = list(range(0, 128)) + list(range(2000, 2050)) + list(range(4096 - 130, 4096))
    run_rows(name, 4096, 4096, 512, seed=31, check_rows=rows)


@pytest.mark.parametrize("name,in_dim", [("q4_k", 512), ("q6_k", 768), ("q8_0", 640)])
@pytest.mark.parametrize("rows,n_tok", [(200, 33), (37, 16), (130, 65)])
def test_gemm_ragged_edges(name, in_dim, rows, n_tok):
    # rows and tokens off the 128 x 64 workgroup tile; Q6_K with 3 blocks a
    # row puts odd rows 2 bytes off a dword; Q8_0 with 20 blocks a row
    run(name, rows, in_dim, n_tok, seed=40 + rows + n_tok)


@pytest.mark.parametrize("in_dim", [128, 384])
def test_gemm_one_and_three_chunks(in_dim):
    # the K loop runs two 128-weight chunks a round: one chunk, and an odd count
    run("q8_0", 130, in_dim, 70, seed=70 + in_dim)


@pytest.mark.parametrize("name", GEMM_TYPES)
def test_matvec_and_gemm_agree_across_the_threshold(name):
    # 15 tokens take the matvec tiles, 16 the GEMM: both match the oracle
    for n_tok in (15, 16):
        run(name, 256, 1024, n_tok, seed=60)


@pytest.mark.parametrize("name", GEMM_TYPES)
def test_gemm_x_range(name):
    # x outside f16's comfortable range, per token: large (|x| ~ 1e5, past
    # f16's 65504), tiny (~1e-6, f16 subnormals), and rows whose 128-weight
    # chunks grow or shrink by 11 orders of magnitude along the row (the
    # running per-token scale).  Each token is checked against its own
    # largest |ref|, so tiny tokens need full relative precision.
    rows, in_dim, n_tok = 130, 1024, 64
    say(f"gemm {name} x range rows={rows} in_dim={in_dim} n_tok={n_tok}")
    ty = oracle.QTYPES[name]
    w = oracle.quant_weights(ty, rows, in_dim, 80)
    x = oracle.normal(81, (n_tok, in_dim)).astype(np.float64)
    ramp = np.logspace(-6, 5, in_dim // 128).repeat(128)
    for t in range(n_tok):
        kind = t % 5
        if kind == 1:
            x[t] *= 1e5
        elif kind == 2:
            x[t] *= 1e-6
        elif kind == 3:
            x[t] *= ramp
        elif kind == 4:
            x[t] *= ramp[::-1]
    x = x.astype(np.float32)
    ref = oracle.matvec(ty, w, rows, in_dim, x)
    y = lmx.matvec(torch.from_numpy(w).cuda(), torch.from_numpy(x).cuda(), qtype=name, rows=rows,
                   in_dim=in_dim)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    assert np.all(np.isfinite(got))
    for t in range(n_tok):
        err = np.abs(got[t] - ref[t]).max()
        scale = np.abs(ref[t]).max()
        assert err <= 3e-5 * scale, f"{name} token {t} (kind {t % 5}): max err {err} vs max |ref| {scale}"
