"""fg_sample_tokens_noalloc (split-draw partials in the library's static device
scratch, no allocation) draws exactly the tokens of fg_sample_tokens with a
caller workspace, on two calls in a row, the second with a smaller input."""
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from flashgrpo_amd import _lib

    return _lib.load()  # argument types from the binding of include/flashgrpo_amd.h


def _noalloc(lib, logits, *, seed, step, seq_ids, draw, temperature, greedy, top_p, row_index=None):
    from flashgrpo_amd import kernels as K

    rows = row_index.numel() if row_index is not None else logits.shape[0]
    out = torch.full((rows,), -7, dtype=torch.int32, device=logits.device)
    rc = lib.fg_sample_tokens_noalloc(logits.data_ptr(), K.dtype_code(logits), logits.stride(0), rows,
                                      logits.shape[1], None if row_index is None else row_index.data_ptr(), None,
                                      None, 0, 0, seed, step, seq_ids.data_ptr(), draw, temperature, int(greedy), 0,
                                      K.top_p_fixed(top_p), out.data_ptr(), K._stream())
    assert rc == 0, lib.fg_last_error()
    return out


@pytest.mark.parametrize("dtype,temperature,greedy,top_p", [
    (torch.bfloat16, 1.0, False, 1.0),    # unrestricted: split max / sum / pick
    (torch.bfloat16, 0.7, False, 0.95),   # split top-p: max, four radix levels, cut, pick
    (torch.float32, 1.0, True, 1.0),      # greedy: split max / pick
    (torch.float32, 1.3, False, 0.9),
])
def test_noalloc_matches_workspace_entry(lib, dtype, temperature, greedy, top_p):
    from flashgrpo_amd import kernels as K

    g = torch.Generator(device="cpu").manual_seed(11)
    # first call: 200 rows of the 7B vocabulary; second: 37 rows of a smaller one
    for call, (rows, V) in enumerate(((200, 152064), (37, 32000))):
        x = (torch.randn(rows, V, generator=g) * 3).to(dtype).to("cuda")
        x[::5, 17] = 40.0  # some dominant rows
        seq = torch.randperm(1000, generator=g)[:rows].to(torch.int32).to("cuda")
        kw = dict(seed=1234 + call, step=3, seq_ids=seq, draw=call, temperature=temperature, greedy=greedy,
                  top_p=top_p)
        got = _noalloc(lib, x, **kw)
        want = K.sample_tokens(x, **kw, split=True)
        torch.cuda.synchronize()
        assert got.tolist() == want.tolist(), (call, rows, V)
        assert got.min().item() >= 0 and got.max().item() < V


def test_noalloc_gathered_rows_then_fewer(lib):
    """row_index gathers (the walk's use) on two calls, the second with fewer rows."""
    from flashgrpo_amd import kernels as K

    g = torch.Generator(device="cpu").manual_seed(5)
    x = torch.randn(64, 152064, generator=g).to(torch.bfloat16).to("cuda")
    for call, rows in enumerate((64, 9)):
        ri = torch.randint(0, 64, (rows,), generator=g).to(torch.int32).to("cuda")
        seq = torch.arange(rows, dtype=torch.int32, device="cuda")
        kw = dict(seed=99, step=call, seq_ids=seq, draw=1, temperature=1.0, greedy=False, top_p=1.0)
        got = _noalloc(lib, x, row_index=ri, **kw)
        want = K.sample_tokens(x, row_index=ri, **kw, split=True)
        torch.cuda.synchronize()
        assert got.tolist() == want.tolist(), call


def test_noalloc_rejects_rows_beyond_its_scratch(lib):
    from flashgrpo_amd import kernels as K

    cap = int(lib.fg_sample_tokens_noalloc_max_rows())
    assert cap == 256
    x = torch.zeros(cap + 1, 64, dtype=torch.float32, device="cuda")
    out = torch.empty(cap + 1, dtype=torch.int32, device="cuda")
    seq = torch.arange(cap + 1, dtype=torch.int32, device="cuda")
    rc = lib.fg_sample_tokens_noalloc(x.data_ptr(), 0, 64, cap + 1, 64, None, None, None, 0, 0, 1, 0,
                                      seq.data_ptr(), 0, 1.0, 0, 0, 0, out.data_ptr(), K._stream())
    assert rc != 0 and b"rows must be in [1, 256]" in lib.fg_last_error()
