"""Host-side behaviour of the reference-API mirror (kvrt.kv_cache,
kvrt.thinker_cache, kvrt.talker) that needs no GPU: bookkeeping, validation
and fail-closed paths, checked against the reference's own known answers
(tests/golden/reference_kats.json) and its tests' fixtures."""
from __future__ import annotations

import json
from pathlib import Path
from types import SimpleNamespace

import pytest
import torch

KATS = json.loads((Path(__file__).resolve().parent / "golden" / "reference_kats.json").read_text())


# ---- thinker_cache -----------------------------------------------------------
@pytest.mark.parametrize("left,right,want", KATS["longest_common_prefix"]["cases"])
def test_longest_common_prefix_matches_reference_answers(left, right, want):
    from kvrt.thinker_cache import longest_common_prefix_length

    assert longest_common_prefix_length(left, right) == want


@pytest.mark.parametrize("prefill,budget,want", KATS["thinker_bucket"]["cases"])
def test_thinker_bucket_matches_reference_answers(prefill, budget, want):
    from kvrt.thinker_cache import select_audio_thinker_cache_bucket

    assert select_audio_thinker_cache_bucket(prefill, budget) == want


def test_thinker_bucket_fails_instead_of_truncating():
    from kvrt.thinker_cache import select_audio_thinker_cache_bucket

    p, b, need = KATS["thinker_bucket"]["overflow"]
    with pytest.raises(ValueError, match=rf"{need}.*4096"):
        select_audio_thinker_cache_bucket(p, b)
    with pytest.raises(ValueError):
        select_audio_thinker_cache_bucket(100, 100, max_cache_len=128)


@pytest.mark.parametrize("prefill,budget", [(0, 1), (-1, 1), (1, 0), (True, 1), (1, 1.5)])
def test_thinker_bucket_rejects_invalid_lengths(prefill, budget):
    from kvrt.thinker_cache import select_audio_thinker_cache_bucket

    with pytest.raises((TypeError, ValueError)):
        select_audio_thinker_cache_bucket(prefill, budget)


def _tiny_static_cache(max_cache_len: int = 8):
    from transformers import PretrainedConfig, StaticCache

    config = PretrainedConfig()
    config.num_hidden_layers = 2
    config.layer_types = ["full_attention", "full_attention"]
    config.sliding_window = None
    config.attention_chunk_size = None
    return StaticCache(config=config, max_cache_len=max_cache_len, max_batch_size=1, device="cpu",
                       dtype=torch.float32)


def test_prefix_copy_fails_closed_when_source_is_too_short():
    """The reference's fixture (test_thinker_cache_prefix.py:69-75): the
    length check fires before any storage is touched."""
    from kvrt.thinker_cache import CachePrefixCopyError, copy_static_cache_prefix

    source = _tiny_static_cache()
    for i in range(2):
        keys = torch.arange(2 * 8, dtype=torch.float32).reshape(1, 2, 2, 4)
        source.update(keys, keys + 1000.0 + i, i)
    target = _tiny_static_cache()
    with pytest.raises(CachePrefixCopyError, match="source cache length"):
        copy_static_cache_prefix(source, target, 3)


def test_prefix_copy_argument_contract():
    from kvrt.thinker_cache import CachePrefixCopyError, copy_static_cache_prefix

    c = _tiny_static_cache()
    with pytest.raises(ValueError):
        copy_static_cache_prefix(c, _tiny_static_cache(), -1)
    with pytest.raises(ValueError):
        copy_static_cache_prefix(c, _tiny_static_cache(), True)
    with pytest.raises(CachePrefixCopyError):
        copy_static_cache_prefix(c, c, 1)
    assert copy_static_cache_prefix(c, _tiny_static_cache(), 0).copied_bytes == 0
    with pytest.raises(CachePrefixCopyError, match="layer"):
        copy_static_cache_prefix(SimpleNamespace(layers=[], get_seq_length=lambda: 4),
                                 SimpleNamespace(layers=[], get_seq_length=lambda: 0), 2)


def test_cpu_static_cache_is_refused_not_copied_on_the_host():
    from kvrt.thinker_cache import CachePrefixCopyError, copy_static_cache_prefix

    source = _tiny_static_cache()
    for i in range(2):
        keys = torch.ones((1, 2, 5, 4))
        source.update(keys, keys, i)
    target = _tiny_static_cache()
    with pytest.raises(CachePrefixCopyError, match="GPU"):
        copy_static_cache_prefix(source, target, 3)
    assert int(target.get_seq_length()) == 0


def test_static_cache_length_and_storage_bytes():
    from kvrt.thinker_cache import static_cache_sequence_length, static_cache_storage_bytes

    c = _tiny_static_cache()
    keys = torch.ones((1, 2, 3, 4))
    for i in range(2):
        c.update(keys, keys, i)
    assert static_cache_sequence_length(c) == 3
    assert static_cache_storage_bytes(c) == 2 * 2 * (1 * 2 * 8 * 4) * 4  # full static capacity


# ---- kv_cache ----------------------------------------------------------------
def test_thinker_context_window_and_budget():
    from kvrt.kv_cache import ThinkerContext

    ctx = ThinkerContext(max_turns=3, max_context_tokens=10)
    for n in (4, 3, 2):
        ctx.add_turn(list(range(n)))
    assert [len(t) for t in ctx.turns] == [4, 3, 2]
    ctx.add_turn([1, 2])  # 4 turns > max_turns: the oldest goes
    assert [len(t) for t in ctx.turns] == [3, 2, 2]
    ctx.add_turn([9] * 6)  # turn count first: [2, 2, 6] is exactly the 10-token budget
    assert [len(t) for t in ctx.turns] == [2, 2, 6]
    ctx.add_turn([9] * 3)  # [2, 6, 3] = 11 tokens: evict oldest first
    assert [len(t) for t in ctx.turns] == [6, 3]
    ctx.add_turn([])
    assert len(ctx.turns) == 2

    tok = SimpleNamespace(encode=lambda s, add_special_tokens=False: [ord(c) for c in s])
    ctx.system_prompt, ctx.summary = "ab", "c"
    assert ctx.flatten(tok) == [97, 98, 99] + ctx.turns[0] + ctx.turns[1]
    msgs = [{"role": "user", "content": str(i)} for i in range(10)]
    ctx.set_messages(msgs)
    assert [m["content"] for m in ctx.messages()] == [str(i) for i in range(4, 10)]
    ctx.clear_turns()
    assert ctx.turns == [] and ctx.messages() == []


def test_kv_seq_len_and_memory_bytes_on_reference_shapes():
    from kvrt.kv_cache import _kv_seq_len, kv_memory_bytes

    pairs = tuple((torch.empty((1, 8, 5, 128), dtype=torch.bfloat16),) * 2 for _ in range(3))
    assert _kv_seq_len(pairs) == 5
    assert _kv_seq_len(None) == 0
    assert _kv_seq_len(SimpleNamespace(get_seq_length=lambda: 7)) == 7
    assert kv_memory_bytes(pairs) == 3 * 2 * 8 * 5 * 128 * 2


def test_prefix_and_turn_state_bookkeeping_with_a_croppable_cache():
    """TurnKVState drives any object with crop/get_seq_length: the turn is
    rolled back to the prefix length recorded at store time."""
    from kvrt.kv_cache import TalkerPrefixKV, TurnKVState

    class Croppable:
        def __init__(self, n):
            self.n = n

        def get_seq_length(self):
            return self.n

        def crop(self, keep):
            self.n = min(self.n, keep)

        def __deepcopy__(self, memo):
            return Croppable(self.n)

    prefix = TalkerPrefixKV()
    assert not prefix.is_ready()
    live = Croppable(12)
    prefix.store(live)
    assert prefix.is_ready() and prefix.seq_len == 12 and prefix.kv is not live
    turn = TurnKVState()
    turn.start_from_prefix(prefix)
    assert turn.prefix_len == 12 and turn.kv is prefix.kv
    live.n = 20
    turn.append(live)
    turn.frames_generated = 8
    turn.truncate_to_position(15)
    assert live.n == 15 and turn.frames_generated == 3
    turn.truncate_to_position(3)  # never below the prefix
    assert live.n == 12
    live.n = 19
    turn.truncate_to_prefix()
    assert live.n == 12 and turn.frames_generated == 0
    turn.clear()
    prefix.clear()
    assert turn.kv is None and not prefix.is_ready() and prefix.seq_len == 0
    empty = TurnKVState()
    empty.start_from_prefix(prefix)
    assert empty.kv is None and empty.prefix_len == 0
    empty.truncate_to_prefix()  # nothing to do


def test_tuple_slicing_refuses_cpu_tensors():
    from kvrt.kv_cache import _clone_kv, _slice_kv

    pairs = ((torch.zeros((1, 1, 4, 64), dtype=torch.bfloat16),) * 2,)
    with pytest.raises(TypeError, match="GPU"):
        _slice_kv(pairs, 2)
    with pytest.raises(TypeError, match="GPU"):
        _clone_kv(pairs)


# ---- talker ------------------------------------------------------------------
def _talker_cache(seq: int = 5):
    pairs = [(torch.zeros((1, 8, seq, 128), dtype=torch.bfloat16), torch.zeros((1, 8, seq, 128), dtype=torch.bfloat16))
             for _ in range(28)]
    layers = [SimpleNamespace(keys=k, values=v) for k, v in pairs]
    return SimpleNamespace(layers=layers, get_seq_length=lambda: seq), pairs


def test_dynamic_cache_view_borrows_the_exact_tensors():
    from kvrt.talker import dynamic_cache_kv_layers

    cache, pairs = _talker_cache()
    seq, layers = dynamic_cache_kv_layers(cache)
    assert seq == 5 and len(layers) == 28
    assert layers[0][0] is pairs[0][0] and layers[-1][1] is pairs[-1][1]


@pytest.mark.parametrize("mutate,message", [
    (lambda c: c.layers.pop(), "28"),
    (lambda c: setattr(c.layers[0], "keys", torch.empty((1, 8, 4, 128), dtype=torch.bfloat16)), "shape"),
    (lambda c: setattr(c.layers[0], "values", torch.empty((1, 8, 5, 128), dtype=torch.float16)), "BF16"),
    (lambda c: setattr(c.layers[0], "keys", torch.empty((1, 8, 5, 256), dtype=torch.bfloat16)), "shape"),
    (lambda c: setattr(c.layers[0], "keys", torch.empty((1, 8, 5, 256), dtype=torch.bfloat16)[:, :, :, ::2]),
     "contiguous"),
    (lambda c: setattr(c, "get_seq_length", lambda: 4), "shape"),
    (lambda c: setattr(c, "get_seq_length", lambda: 0), "at least one"),
])
def test_dynamic_cache_view_fails_closed(mutate, message):
    """The reference's cases (test_qwen_native_audio_q1.py:52-68)."""
    from kvrt.talker import dynamic_cache_kv_layers

    cache, _ = _talker_cache()
    mutate(cache)
    with pytest.raises(ValueError, match=message):
        dynamic_cache_kv_layers(cache)


def test_audio_q1_counter_advances_then_fails_closed():
    from kvrt.talker import advance_audio_q1_position

    kat = KATS["audio_q1_counter"]
    start, limit = kat["start"], kat["start"] + kat["frames"]
    pos = start
    for off in range(1, kat["frames"] + 1):
        pos = advance_audio_q1_position(pos, limit)
        assert pos == start + off
    with pytest.raises(RuntimeError, match="limit"):
        advance_audio_q1_position(pos, limit)
    with pytest.raises(RuntimeError):
        advance_audio_q1_position(-1, 5)


@pytest.mark.parametrize("kwargs,ok", [
    (dict(prefix_attention_mode=3), False),                                   # native_qwen_talker.py:1211
    (dict(prefix_log_gate=float("inf")), False),
    (dict(prefix_attention_mode=2, visible_prefix_count=0), False),           # :1213
    (dict(prefix_attention_mode=2, visible_prefix_count=3), True),
    (dict(prefix_position=8), False),                                         # inside the audio region
    (dict(prefix_position=1), False),                                         # before the prefix start
    (dict(audio_position=7), False),
    (dict(), True),
])
def test_talker_mask_validation(kwargs, ok):
    from kvrt import TalkerMask

    args = dict(prefix_start=2, audio_start=8, prefix_position=4, audio_position=10)
    args.update(kwargs)
    if ok:
        c = TalkerMask(**args).to_c()
        assert (c.prefix_start, c.audio_start, c.prefix_position, c.audio_position) == (
            args["prefix_start"], args["audio_start"], args["prefix_position"], args["audio_position"])
    else:
        with pytest.raises(ValueError):
            TalkerMask(**args)
