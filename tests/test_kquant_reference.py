"""Why the K-quants have no device GEMV: the compiled reference's own
gguf_dequant (/root/reference/src/l2_codec.c:84-199), which matmul_q's
fallback (:350-366) runs on every row of a K-quant matrix, does not define
its output.

  * Q3_K, Q4_K, Q5_K, Q6_K write only part of each 256-element block
    (deq_q3_K :107-127, deq_q4_K :129-145 and deq_q5_K :147-164 loop
    n += 64 with l < 32; deq_q6_K :166-183 n += 128 with outputs n+l and
    n+l+32 only): the rest of the row keeps whatever the fallback's row
    buffer held - a per-thread malloc reused across rows.  Shown by running
    it twice over two different fills of the output: the unwritten elements
    keep each fill.
  * Q2_K (:85-105) reads q[j*32 + l] for j < 4 (128 bytes per half block,
    where a block holds 64): its output depends on the bytes after the block.
  * Q8_K has no case: zeros (and a message on stderr).

The device refuses these types (G2B_EUNSUP; include/g2b_matmul.h), as
test_matmul_oracle.test_row_bytes checks for the row size."""
import numpy as np
import pytest

from helpers import require_ref
from oracle import orc

KQ_BYTES = {orc.T_Q2_K: 84, orc.T_Q3_K: 110, orc.T_Q4_K: 144, orc.T_Q5_K: 176,
            orc.T_Q6_K: 210, orc.T_Q8_K: 292}


def block(t, seed, extra=512):
    """One K-quant block of random bytes with an fp16 scale of 1/64 at every
    place a scale may sit, followed by `extra` random bytes."""
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, KQ_BYTES[t] + extra, dtype=np.uint8)
    one = np.array([1.0 / 64], np.float16).view(np.uint8)
    for off in (0, 2, 80, 82, 108, 208):  # d / dmin of each layout
        if off + 2 <= KQ_BYTES[t]:
            b[off:off + 2] = one
    return b


@pytest.mark.parametrize("t,written", [(orc.T_Q3_K, 128), (orc.T_Q4_K, 128),
                                       (orc.T_Q5_K, 128), (orc.T_Q6_K, 128)])
def test_kquant_dequant_leaves_elements_unwritten(t, written):
    require_ref()
    src = block(t, 100 + t)
    fills = (np.float32(1234.5), np.float32(-777.25))
    outs = []
    for f in fills:
        out = np.full(256, f, np.float32)
        orc.ref_gguf_dequant(t, src, out, 256)
        outs.append(out)
    kept = (outs[0] == fills[0]) & (outs[1] == fills[1])
    assert int(kept.sum()) == 256 - written, int(kept.sum())
    # where it does write, the two runs agree
    assert np.array_equal(outs[0][~kept].view(np.uint32), outs[1][~kept].view(np.uint32))


def test_q2k_dequant_reads_past_its_block():
    require_ref()
    a = block(orc.T_Q2_K, 7)
    b = a.copy()
    b[KQ_BYTES[orc.T_Q2_K]:] = np.random.default_rng(8).integers(0, 256, 512, dtype=np.uint8)
    oa, ob = np.zeros(256, np.float32), np.zeros(256, np.float32)
    orc.ref_gguf_dequant(orc.T_Q2_K, a, oa, 256)
    orc.ref_gguf_dequant(orc.T_Q2_K, b, ob, 256)
    assert not np.array_equal(oa, ob)  # same 84 block bytes, different output


def test_q8k_dequant_has_no_case():
    require_ref()
    out = np.full(256, np.float32(3.0), np.float32)
    orc.ref_gguf_dequant(orc.T_Q8_K, block(orc.T_Q8_K, 3), out, 256)
    assert not out.any()
