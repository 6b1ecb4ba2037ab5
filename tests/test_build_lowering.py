"""The build's check of the coherent-access lowering, without a GPU: the
helpers of kvrt_device.h that the single-launch decode merge exchanges its
partials and arrival counts through compile (alone, in
kvrt_coherence_probe.hip, with the library's flags) to device-scope stores and
loads (sc1) and an L2 atomic add, and the checker refuses a listing in which
any of them differs: a store or load without its scope bit, an L2 write-back
or invalidate around an access, a missing probe kernel."""
from __future__ import annotations

import re
import shutil

import pytest

from kvrt import _build as B

pytestmark = pytest.mark.skipif(shutil.which("hipcc") is None and not B.Path("/opt/rocm/bin/hipcc").exists(),
                                reason="hipcc not available")


@pytest.fixture(scope="module")
def asm() -> str:
    return B.coherence_probe_asm()


def test_coherent_helpers_lower_as_the_merge_requires(asm):
    assert B.coherence_errors(asm) == []
    ops = B.memory_ops(asm)
    assert ops["kvrt_probe_store16"] == [("global_store_dwordx2", {"sc1"})] * 2
    assert ops["kvrt_probe_arrive"][0] == ("global_atomic_add", {"sc0"})
    B.check_coherence_lowering()  # what build() runs


def _in_kernel(asm: str, name: str, pattern: str, repl: str) -> str:
    """asm with the first match of pattern inside kernel `name` replaced."""
    start = asm.index(f"\n{name}:")
    end = asm.index("s_endpgm", start)
    body, n = re.subn(pattern, repl, asm[start:end], count=1)
    assert n == 1, (name, pattern)
    return asm[:start] + body + asm[end:]


@pytest.mark.parametrize("name,pattern,repl", [
    ("kvrt_probe_store16", r"(offset:8) sc1", r"\1"),  # second half left in the L2
    ("kvrt_probe_store_f32", r" sc1", r" nt"),
    ("kvrt_probe_load_f32x2", r"(global_load_dwordx2 [^\n]*) sc1", r"\1"),  # a load that may hit a stale L2 line
    ("kvrt_probe_load_f32", r"global_load_dword ", "global_load_dwordx2 "),
    ("kvrt_probe_arrive", r"(\tglobal_atomic_add)", "\tbuffer_wbl2 sc1\n\\1"),  # release lowering appeared
    ("kvrt_probe_clear", r"global_store_dword [^\n]*sc1", "global_store_dword v0, v1, s[0:1] sc0 sc1"),
])
def test_checker_refuses_a_changed_lowering(asm, name, pattern, repl):
    bad = _in_kernel(asm, name, pattern, repl)
    errs = B.coherence_errors(bad)
    assert errs and all(e.startswith(name) for e in errs), errs


def test_checker_refuses_a_missing_probe_kernel(asm):
    bad = asm.replace("\nkvrt_probe_clear:", "\nkvrt_probe_renamed:")
    assert [e for e in B.coherence_errors(bad) if e.startswith("kvrt_probe_clear: not found")]
