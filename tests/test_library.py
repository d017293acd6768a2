"""The C-ABI library loads and exports every symbol include/specdec.h declares
(no GPU needed: nothing is launched)."""
import re
from pathlib import Path

from specdec import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "specdec.h"


def declared() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"^int (specdec_\w+)\(", text, flags=re.M))


def test_header_and_binding_agree():
    assert declared() == set(_lib.SIGNATURES)


def test_library_exports_every_symbol():
    lib = _lib.load()
    for name in declared():
        assert hasattr(lib, name), name
    assert lib.specdec_abi_version() == _lib.ABI_VERSION


def test_attention_workspace_query_needs_no_gpu():
    import ctypes

    lib = _lib.load()
    floats = ctypes.c_int64()
    # B=1, T=5, 32/32 heads, d=64, 4101 keys: one tile per head, 9 splits of 512
    assert lib.specdec_attention_workspace(1, 5, 32, 32, 64, 4101, 0, ctypes.byref(floats)) == 0
    assert floats.value == 32 * 9 * 16 * 65
    assert lib.specdec_attention_split(1, 5, 32, 32, 4101) == 512
    assert lib.specdec_attention_workspace(1, 5, 32, 32, 128, 10, 0, ctypes.byref(floats)) == 3


def test_invalid_arguments_are_rejected_before_launch():
    lib = _lib.load()
    # negative sizes and null pointers return SPECDEC_EINVAL without touching a device
    assert lib.specdec_probabilities(None, 0, -1, 10, 10, 1.0, None, 10, None, 0, None) == 1
    assert lib.specdec_ngram_lookup(None, 0, None, 1, 4, 9, None, None, None) == 1  # null pointers
    assert lib.specdec_block_plan(None, 1, None, None, 4, 5, None, 1, 0, None, None) == 1  # top > num_blocks


def test_attention_entry_points_check_token_strides_before_launch():
    lib = _lib.load()
    fake = 1 << 20  # never dereferenced: the call returns before any launch
    # q [tokens, 32 heads x 64], out likewise: a token stride shorter than a
    # token's heads would make rows overlap -- invalid
    def call(q_stride, out_stride):
        return lib.specdec_paged_attention(fake, 2, q_stride, fake, fake, fake, 8, fake, 1, 5, 32, 32, 64, 16, 0.125,
                                           64, 0, fake, 1 << 20, fake, out_stride, None)
    assert call(32 * 64 - 8, 32 * 64) == 1
    assert call(32 * 64, 32 * 64 - 8) == 1
    # with rope the rows are qkv rows: (32 + 2 x 32) x 64 elements
    assert lib.specdec_rope_paged_attention(fake, 2, 32 * 64, fake, fake, None, 0, 0.0, fake, fake, fake, 8, fake, 1,
                                            5, 32, 32, 64, 16, 0.125, 64, 0, fake, 1 << 20, fake, 32 * 64,
                                            None) == 1


def test_head_entry_points_check_shapes_before_launch():
    import ctypes

    lib = _lib.load()
    nbytes = ctypes.c_int64()
    assert lib.specdec_head_workspace(ctypes.byref(nbytes)) == 0 and nbytes.value > 0
    # hidden not a multiple of 32: unsupported; a negative row count: invalid
    assert lib.specdec_head_logits(16, 48, 16, 48, 1, 48, 100, 16, 100, None) == 3
    assert lib.specdec_head_logits(16, 64, 16, 64, -1, 64, 100, 16, 100, None) == 1
    # more than 16 rows in one fused call
    assert lib.specdec_head_probabilities(16, 64, 16, 64, 17, 64, 100, 1.0, 16, 100, None, 0, None, 0, 16,
                                          nbytes.value, 0, None) == 3


def test_spin_wait_is_a_plain_request():
    """specdec.spin_wait() asks HIP to spin while waiting and reports whether
    HIP took it (in a fresh process: it must come before any GPU use; with
    no GPU HIP refuses it)."""
    import subprocess
    import sys
    from pathlib import Path

    pkg = Path(__file__).resolve().parents[1] / "speculative-decoder_amd"
    out = subprocess.run([sys.executable, "-c", "import specdec; print(specdec.spin_wait())"], cwd=pkg,
                         capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    assert out.stdout.strip() in ("True", "False")


def test_accept_entry_points_check_shapes_before_launch():
    import ctypes

    lib = _lib.load()
    nbytes = ctypes.c_int64()
    # arrival counters, the epoch and padding (16 words), then per row the
    # meeting words: 2 + 2 per chunk, 2 per logit row (<= 33) and chunk, 64 chunks
    assert lib.specdec_accept_workspace(3, ctypes.byref(nbytes)) == 0
    assert nbytes.value == (16 + 3 * (4 * 64 + 2 * 33 * 64)) * 8
    # the logits form: more than 16 drafted positions, or bf16 logits, are
    # unsupported; a negative temperature is invalid (no pointer is touched)
    fake, ws = 1 << 20, 1 << 24
    args = lambda dtype, temp, k: (fake, fake, dtype, (k + 1) * 64, 64, k * 64, 64, temp, fake, fake, fake, 1, k, 64,
                                   fake, ws, nbytes.value, 0, None)
    assert lib.specdec_accept_reject_logits(*args(0, 1.0, 17)) == 3
    assert lib.specdec_accept_reject_logits(*args(2, 1.0, 4)) == 3
    assert lib.specdec_accept_reject_logits(*args(0, -1.0, 4)) == 1


def test_verdict_is_the_reference_two_field_dataclass():
    import dataclasses

    import torch

    from spec.accept import Verdict, host_draft

    assert [f.name for f in dataclasses.fields(Verdict)] == ["n_accepted", "next_token"]
    v = Verdict(torch.tensor([1]), torch.tensor([2]))
    assert host_draft(v) is None and len(dataclasses.astuple(v)) == 2
    with __import__("pytest").raises(dataclasses.FrozenInstanceError):
        v.n_accepted = torch.tensor([0])
