"""Host-side contracts of the entry points (no GPU): contract violations raise ValueError
before any launch, round-state violations raise RuntimeError, and ineligible sparse-target
batches return None -- the error behaviour of the reference's wrappers."""

from types import SimpleNamespace

import pytest
import torch


def _chain_args(bs=3, k=16, width=16):
    """tests/test_sampled_confidence.py:11-31 (CPU tensors)."""
    n = bs * (width - 1)
    table = torch.randn((n, k, k)) * 2
    candidates = torch.arange(k).expand(n, k).contiguous()
    greedy = torch.zeros(bs, dtype=torch.int32)
    return (table, torch.full((bs,), 1.0), torch.tensor([3, k, 7], dtype=torch.int32).repeat(bs)[:bs],
            torch.tensor([0.65, 0.95, 1.0]).repeat(bs)[:bs], torch.tensor([0.05, 0.0, 0.2]).repeat(bs)[:bs],
            greedy, torch.rand(n), candidates, candidates[:, 0].clone(), torch.empty(n, dtype=torch.int64),
            torch.empty((n, k)), width)


@pytest.mark.parametrize("invalid", ["dtype", "capacity", "strided", "device"])
def test_serial_chain_confidence_contract(invalid):
    """tests/test_sampled_confidence.py:59-70."""
    from dspine_amd.kernels.dspine import serial_sample_chain

    args = _chain_args()
    n = 3 * 15
    confidence = {
        "dtype": lambda: torch.empty(n, dtype=torch.float64),
        "capacity": lambda: torch.empty(n - 1),
        "strided": lambda: torch.empty(n * 2)[::2],
        "device": lambda: torch.empty(n, device="meta"),
    }[invalid]()
    with pytest.raises(ValueError, match="confidence needs contiguous float32"):
        serial_sample_chain(*args, confidence_out=confidence)


def test_serial_chain_layout_and_dtypes():
    from dspine_amd.kernels.dspine import serial_sample_chain

    args = list(_chain_args())
    bad = list(args)
    bad[0] = args[0][:-1]
    with pytest.raises(ValueError, match="table layout"):
        serial_sample_chain(*bad)
    bad = list(args)
    bad[2] = args[2].to(torch.int64)
    with pytest.raises(ValueError, match="dtype contract"):
        serial_sample_chain(*bad)
    bad = list(args)
    bad[10] = torch.empty((3, 16))
    with pytest.raises(ValueError, match="output buffers"):
        serial_sample_chain(*bad)


def _sparse_kwargs(bs=2):
    out = (torch.empty(bs, dtype=torch.int32), torch.empty(bs, dtype=torch.int32), torch.empty(bs, dtype=torch.int64),
           torch.empty((bs, 16), dtype=torch.int64), torch.empty(bs, dtype=torch.int32))
    return dict(candidates=torch.zeros((bs, 16), dtype=torch.int64), dense_p=torch.zeros((bs * 16, 97)),
                packed=None, q_ids=torch.zeros((bs, 15, 16), dtype=torch.int32), q_values=torch.zeros((bs, 15, 16)),
                verify_lens=torch.full((bs,), 16, dtype=torch.int32), uniforms=torch.zeros((bs, 15)),
                uniform_final=torch.zeros(bs), prefix_lens=torch.zeros(bs, dtype=torch.int32), outputs=out)


def test_accept_sparse_contract():
    """sampling/sparse/accept.py:483-511."""
    from dspine_amd.sampling.sparse.accept import accept_sparse

    kw = _sparse_kwargs()
    with pytest.raises(ValueError, match="Pure packed rejection requires packed"):
        accept_sparse(torch, **{**kw, "dense_p": None})
    packed = (torch.zeros((32, 8), dtype=torch.int32), torch.zeros((32, 8)), torch.zeros(32, dtype=torch.int32),
              torch.zeros(32, dtype=torch.int32))
    with pytest.raises(ValueError, match="normalized packed"):
        accept_sparse(torch, **{**kw, "dense_p": None, "packed": packed}, vocab_size=97, raw_fallback=True)
    with pytest.raises(ValueError, match="vocab_size differs"):
        accept_sparse(torch, **kw, vocab_size=98)
    with pytest.raises(ValueError, match="denominator"):
        accept_sparse(torch, **kw, raw_fallback=True)
    with pytest.raises(ValueError, match="row_offsets"):
        accept_sparse(torch, **kw, row_offsets=torch.zeros(3, dtype=torch.int32))
    with pytest.raises(ValueError, match="row_offsets"):
        accept_sparse(torch, **kw, row_offsets=torch.zeros(2, dtype=torch.float32))


def test_capped_chain_contract():
    """sampling/rejection.py:111-135."""
    from dspine_amd.sampling.rejection import sample_capped_chain_from_probs

    bs, V = 2, 50
    out = (torch.empty(bs, dtype=torch.int32), torch.empty(bs, dtype=torch.int32), torch.empty(bs, dtype=torch.int64),
           torch.empty((bs, 16), dtype=torch.int64), torch.empty(bs, dtype=torch.int32))
    kw = dict(candidates=torch.zeros((bs, 16), dtype=torch.int64), target_probs=torch.zeros((bs, 16, V)),
              draft_probs=torch.zeros((bs, 15, V)), verify_lens=torch.full((bs,), 16, dtype=torch.int32),
              uniforms=torch.zeros((bs, 15)), uniform_final=torch.zeros(bs),
              prefix_lens=torch.zeros(bs, dtype=torch.int32), outputs=out)
    with pytest.raises(ValueError, match="target"):
        sample_capped_chain_from_probs(**{**kw, "target_probs": torch.zeros((bs, 15, V))})
    with pytest.raises(ValueError, match="draft q"):
        sample_capped_chain_from_probs(**{**kw, "draft_probs": torch.zeros((bs, 16, V))})
    with pytest.raises(ValueError, match="cap or uniform"):
        sample_capped_chain_from_probs(**{**kw, "uniforms": torch.zeros((bs, 16))})
    with pytest.raises(ValueError, match="final uniform"):
        sample_capped_chain_from_probs(**{**kw, "prefix_lens": torch.zeros(bs + 1, dtype=torch.int32)})
    with pytest.raises(ValueError, match="Expected accept"):
        sample_capped_chain_from_probs(**{**kw, "outputs": out[:4]})
    with pytest.raises(ValueError, match="contiguous"):
        sample_capped_chain_from_probs(**{**kw, "target_probs": torch.zeros((bs, V, 16)).transpose(1, 2)})
    with pytest.raises(ValueError, match="device"):
        sample_capped_chain_from_probs(**kw)  # CPU tensors: the HIP path needs device tensors


def test_sparse_target_eligibility():
    """sampling/sparse/target.py:106-116: unsupported batches return None before any work."""
    from dspine_amd.sampling.sparse.target import build_sparse_target

    info = SimpleNamespace(temperatures=torch.ones(2, 1), top_ks=torch.tensor([5, 8], dtype=torch.int32),
                           top_ps=torch.ones(2), min_ps=torch.zeros(2), need_min_p_sampling=False,
                           is_any_greedy=False, max_top_k=8)
    logits = torch.zeros(32, 100)
    assert build_sparse_target(logits, info, sampling_backend="pytorch") is None
    assert build_sparse_target(logits, SimpleNamespace(**{**vars(info), "need_min_p_sampling": True})) is None
    assert build_sparse_target(logits, SimpleNamespace(**{**vars(info), "is_any_greedy": True})) is None
    assert build_sparse_target(logits, SimpleNamespace(**{**vars(info), "max_top_k": None})) is None
    assert build_sparse_target(logits, SimpleNamespace(**{**vars(info), "max_top_k": 33})) is None
    with pytest.raises(ValueError, match="rows,vocab"):
        build_sparse_target(logits[None], info)


def test_worker_refuses_stale_rounds():
    """runtime/worker.py:1030-1037 and sampling/target.py:45-49."""
    from dspine_amd.runtime import worker as Wk

    Wk.set_active_worker(None)
    with pytest.raises(RuntimeError, match="before the DSpine worker exists"):
        Wk.accept_dspine_sampled_round(candidates=torch.zeros((2, 16), dtype=torch.int64),
                                       next_token_logits=torch.zeros(32, 10), sampling_info=None)
    wk = Wk.VerifyWorker(16, "cpu")
    Wk.set_active_worker(wk)
    try:
        with pytest.raises(RuntimeError, match="without this round's sampled draft chain"):
            Wk.accept_dspine_sampled_round(candidates=torch.zeros((2, 16), dtype=torch.int64),
                                           next_token_logits=torch.zeros(32, 10), sampling_info=None)
        wk._dspine_sampler.stage(torch.zeros((3, 15, 16), dtype=torch.int64), torch.zeros((3, 15, 16)))
        with pytest.raises(RuntimeError, match="staged round has batch 3"):
            Wk.accept_dspine_sampled_round(candidates=torch.zeros((2, 16), dtype=torch.int64),
                                           next_token_logits=torch.zeros(32, 10), sampling_info=None)
        with pytest.raises(RuntimeError, match="this round's actual proposal q"):
            wk.target_distribution.sample_prefix(candidates=torch.zeros((2, 16), dtype=torch.int64),
                                                 next_token_logits=torch.zeros(32, 10), sampling_info=None,
                                                 prefix_lens=torch.zeros(2, dtype=torch.int32), bs=2,
                                                 verify_lens=torch.full((2,), 16, dtype=torch.int32))
    finally:
        Wk.set_active_worker(None)


def test_dspine_accept_sampling_layout():
    """runtime/worker.py:529-534."""
    from dspine_amd.runtime.worker import dspine_accept_sampling

    with pytest.raises(RuntimeError, match="candidate / q layout"):
        dspine_accept_sampling(candidates=torch.zeros((2, 16), dtype=torch.int64), target_logits=None,
                               candidate_ids=torch.zeros((2, 14, 16), dtype=torch.int64),
                               q_rows=torch.zeros((2, 14, 16)), sampling_info=None, sampling_backend="pytorch",
                               dense_q=None)


def test_filter_without_flags_returns_the_input_view():
    """runtime/worker.py:477-478: no filter flag -> the unnormalised input, unchanged."""
    from dspine_amd.runtime.worker import filter_target_probs

    probs = torch.rand(6, 11)
    info = SimpleNamespace(need_top_k_sampling=False, need_top_p_sampling=False, need_min_p_sampling=False)
    out = filter_target_probs(probs, info, 3, 2, "pytorch")
    assert out.shape == (2, 3, 11) and out.data_ptr() == probs.data_ptr()


def test_compress_and_padding_need_device_tensors():
    from dspine_amd.sampling.padding import logits_padding
    from dspine_amd.sampling.sparse.accept import compress_probs

    with pytest.raises(ValueError):
        compress_probs(torch, torch.zeros(2, 5, dtype=torch.float64))
    with pytest.raises(ValueError, match="device"):
        compress_probs(torch, torch.zeros(2, 5))
    with pytest.raises(ValueError, match="device"):
        logits_padding(None, torch.zeros(1), (2, 5))
