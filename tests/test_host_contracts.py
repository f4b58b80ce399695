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


def test_sample_prefix_route_rule():
    """The sparse joint route (sampling/target.py:53-66, sparse/target.py:106-116): the host rule
    and the oracle's restatement agree, and each condition alone turns it off."""
    import oracle.verify_oracle as O
    from dspine_amd import workloads as W
    from dspine_amd.sampling.target import sparse_route

    info = W.sampling_info([1.0, 0.6], [20, 8], [0.95, 1.0])
    for backend, vocab, K in (("flashinfer", 1000, 16), ("pytorch", 1000, 16), ("flashinfer", 1000, 8),
                              ("flashinfer", 10, 16)):
        assert sparse_route(info, backend, vocab, K) == O.sparse_route(info, backend, vocab, K)
    assert sparse_route(info, "flashinfer", 1000, 16)
    assert not sparse_route(info, "flashinfer", 10, 16)  # max top-k above the vocabulary
    for bad in (W.sampling_info([1.0, 0.0], [20, 8], [0.95, 1.0]),               # a greedy row
                W.sampling_info([1.0, 0.6], [20, 0], [0.95, 1.0]),               # top-k off
                W.sampling_info([1.0, 0.6], [20, 8], [0.95, 1.0], [0.1, 0.0]),   # min-p
                W.sampling_info([1.0, 0.6], [40, 8], [0.95, 1.0])):              # top-k above 32
        assert not sparse_route(bad, "flashinfer", 1000, 16)
        assert not O.sparse_route(bad, "flashinfer", 1000, 16)


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


# ------------------------------------------------------------------------------------------
# the AROUND hook on the verify-logit adjustments (sampling/compact.py:82-116)
# ------------------------------------------------------------------------------------------
class _Info(list):
    """A sampling_info with no adjustment tensors (adjust_logits is then a no-op) and
    len() = batch size."""

    def __init__(self, bs, custom=False):
        super().__init__(range(bs))
        self.has_custom_logit_processor = custom


@pytest.fixture
def hook_env(monkeypatch):
    import sys
    import types

    from dspine_amd.runtime import worker as Wk

    calls = []
    sampler_mod = types.ModuleType("sglang.srt.layers.sampler")
    sampler_mod.apply_custom_logit_processor = lambda logits, info, num_tokens_in_batch: calls.append(
        ("custom", logits.shape, num_tokens_in_batch))
    for name in ("sglang", "sglang.srt", "sglang.srt.layers"):
        monkeypatch.setitem(sys.modules, name, types.ModuleType(name))
    monkeypatch.setitem(sys.modules, "sglang.srt.layers.sampler", sampler_mod)
    monkeypatch.setattr(Wk, "_active_worker", None)

    def original(**kw):
        calls.append(("original", kw["next_token_logits"].shape, kw["draft_token_num"]))
        return "original"

    return Wk, calls, original


def test_hook_without_worker_runs_original(hook_env):
    from dspine_amd.sampling.compact import around_verify_logits_adjustments

    Wk, calls, original = hook_env
    logits = torch.zeros(6, 5)
    assert around_verify_logits_adjustments(original, next_token_logits=logits, sampling_info=_Info(2),
                                            draft_token_num=3) == "original"
    assert calls == [("original", (6, 5), 3)]


def test_hook_worker_without_controller_adjusts_full_block(hook_env):
    from dspine_amd.sampling.compact import around_verify_logits_adjustments

    Wk, calls, original = hook_env
    Wk._active_worker = SimpleNamespace(verify_caps=None)
    logits = torch.zeros(6, 5)
    assert around_verify_logits_adjustments(original, next_token_logits=logits, sampling_info=_Info(2),
                                            draft_token_num=3) is None
    assert calls == []  # neither the original nor a custom processor
    # custom logit processors run before the DSpine adjustments, over the [bs*T, V] rows
    around_verify_logits_adjustments(original, next_token_logits=logits, sampling_info=_Info(2, custom=True),
                                     draft_token_num=3)
    assert calls == [("custom", (6, 5), 3)]
    assert around_verify_logits_adjustments(original, next_token_logits=logits, sampling_info=None,
                                            draft_token_num=3) is None
    with pytest.raises(ValueError, match="request/block layout"):
        around_verify_logits_adjustments(original, next_token_logits=logits, sampling_info=_Info(3),
                                         draft_token_num=3)
    with pytest.raises(ValueError, match="positive draft width"):
        around_verify_logits_adjustments(original, next_token_logits=logits, sampling_info=_Info(2),
                                         draft_token_num=0)


def test_hook_compact_round(hook_env):
    from dspine_amd.sampling.compact import around_verify_logits_adjustments

    Wk, calls, original = hook_env
    packed = torch.zeros(4, 5)
    ctl = SimpleNamespace(compact_round=True, compact_logits=packed, row_to_request=torch.tensor([0, 0, 1, 1]))
    Wk._active_worker = SimpleNamespace(verify_caps=ctl)
    with pytest.raises(RuntimeError, match="do not belong to this round"):
        around_verify_logits_adjustments(original, next_token_logits=packed.clone(), sampling_info=_Info(2),
                                         draft_token_num=3)
    # the round's own packed rows: adjusted with the controller's row map (no custom step)
    assert around_verify_logits_adjustments(original, next_token_logits=packed,
                                            sampling_info=_Info(2, custom=True), draft_token_num=3) is None
    assert calls == []
    # a controller outside a compact round: the full-block branch
    ctl.compact_round = False
    around_verify_logits_adjustments(original, next_token_logits=torch.zeros(6, 5),
                                     sampling_info=_Info(2, custom=True), draft_token_num=3)
    assert calls == [("custom", (6, 5), 3)]


# ------------------------------------------------------------------------------------------
# controller acceptance state checks (verification/caps.py:331-379, ragged.py:282-335)
# ------------------------------------------------------------------------------------------
def _accept_kwargs(bs=2, T=4):
    return dict(candidates=torch.zeros(bs, T, dtype=torch.int64), next_token_logits=torch.zeros(bs * T, 8),
                sampling_info=None, draft_input=None, prefix_lens=torch.zeros(bs, dtype=torch.int32), bs=bs)


def test_capped_accept_requires_confirmed_forward():
    from dspine_amd.verification import caps

    ctl = SimpleNamespace(executed_width=3, active=2, sampled_round=False, full=4)
    with pytest.raises(RuntimeError, match="confirmed shortened target forward"):
        caps.accept(ctl, **_accept_kwargs())


def test_ragged_accept_requires_confirmed_packed_verification():
    from dspine_amd.verification import ragged

    ctl = SimpleNamespace(ragged_round=True, batch_size=2, executed_tokens=5, tokens=6, sampled_round=False,
                          full=4)
    with pytest.raises(RuntimeError, match="confirmed packed verification"):
        ragged.accept(ctl, **_accept_kwargs())
    ctl.executed_tokens = 6
    with pytest.raises(RuntimeError, match="confirmed packed verification"):
        ragged.accept(ctl, **_accept_kwargs(bs=3))
    # not a ragged round: the capped controller's checks apply
    ctl = SimpleNamespace(ragged_round=False, executed_width=4, active=3, sampled_round=False, full=4)
    with pytest.raises(RuntimeError, match="confirmed shortened target forward"):
        ragged.accept(ctl, **_accept_kwargs())


def test_sample_prefix_compact_rows_need_offsets():
    from dspine_amd.sampling.target import TargetDistribution

    sampler = SimpleNamespace(round_sampled=True, round_bs=2)
    td = TargetDistribution(SimpleNamespace(block_size=4, _dspine_sampler=sampler))
    with pytest.raises(ValueError, match="need their row_offsets"):
        td.sample_prefix(candidates=torch.zeros(2, 4, dtype=torch.int64), next_token_logits=torch.zeros(5, 8),
                         sampling_info=None, prefix_lens=torch.zeros(2, dtype=torch.int32), bs=2,
                         verify_lens=torch.tensor([2, 3], dtype=torch.int32),
                         row_to_request=torch.tensor([0, 0, 1, 1, 1]))


# ------------------------------------------------------------------------------------------
# SPS planner contracts (verification/sps.py:35-70)
# ------------------------------------------------------------------------------------------
def test_sps_plan_contracts():
    from dspine_amd.verification.sps import allocate_verify_lens, device_plan

    raw, table, depth = torch.rand(3, 15), torch.rand(15, 8), torch.arange(15)
    cfg = SimpleNamespace(min_verify_len=1, survival_eps=0.0)
    with pytest.raises(ValueError, match="SPS budget"):
        allocate_verify_lens(raw, table, depth, 2)
    with pytest.raises(ValueError, match="SPS budget"):
        device_plan(raw, table, depth, 49, cfg)
    with pytest.raises(ValueError, match="one root per request"):
        device_plan(raw, table, depth, 10, SimpleNamespace(min_verify_len=2, survival_eps=0.0))
    with pytest.raises(ValueError, match="one root per request"):
        device_plan(raw, table, depth, 10, SimpleNamespace(min_verify_len=1, survival_eps=0.1))
    with pytest.raises(ValueError, match="graph tier"):
        device_plan(raw, table, depth, 10, cfg, graph_tokens=12)
    with pytest.raises(ValueError, match="one table row per draft position"):
        allocate_verify_lens(raw, table, depth[:-1], 10)
    with pytest.raises(ValueError, match="at most bins - 1"):
        allocate_verify_lens(raw, table, depth, 10, torch.linspace(0.1, 0.9, 8, dtype=torch.float64))
    with pytest.raises(ValueError, match="device"):  # CPU tensors never reach the HIP library
        allocate_verify_lens(raw, table, depth, 10)


def test_proposal_capture_sizes_and_factor_contracts():
    """graph.py's capture-size rule (sizes that at least double, the largest configured size
    closing the list) and factor_table's contract checks before any launch."""
    from dspine_amd.sampling.factorized.graph import _capture_sizes
    from dspine_amd.sampling.factorized.kernels import factor_table

    assert _capture_sizes([1, 2, 4, 8, 16, 32], 33) == [1, 2, 4, 8, 16, 32]
    assert _capture_sizes([1, 3, 5, 6, 12, 13], 12) == [1, 3, 6, 12]
    assert _capture_sizes([4, 5, 7], 64) == [7]  # the largest replaces the last kept size
    assert _capture_sizes([0, 100], 64) == []
    raw = torch.zeros(32, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="bs \\* \\(t - 1\\)"):
        factor_table(raw, torch.ones(32), torch.zeros(32, 8, dtype=torch.bfloat16), torch.zeros(2, dtype=torch.int64),
                     torch.zeros(29, 16, dtype=torch.int64), {}, 1e-6, 16, None, None, None)
