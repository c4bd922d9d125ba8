"""Both LM heads at hidden widths other than the model's 896 (GPU).

The GEMMs' block loops treat the first blocks and the last ones apart: the
first block starts the running totals, loads run one (Q4_0) or two (Q8_0)
blocks ahead, and an odd or short block count ends outside the loop.  The
model's width (28 blocks) exercises none of the short or odd cases, so each
head runs here at 1, 2, 3, 5 and 29 blocks, through the narrow kernel with
its own quantisation (1 and 3 rows), the narrow kernel after lm_quant_kernel
(9 rows) and the wide kernel (66 rows).  Logits must be bit-identical to the
oracle's restatement of inference_q4_matvec_rows_prepared /
inference_q8_matvec_rows_prepared (fp32_sse2.rs:1217-1248, 1251-1280), and the
draws identical to the oracle sampler's on those logits.  At the odd widths
one Q4_0 tile carries an infinite weight scale (the subtract-then-multiply
epilogue); every row then ends in the same error record as the oracle's.
"""
import numpy as np
import pytest

from oracle import oracle as o
from promptboot_amd import sampler as s
from tests.conftest import to_dev

pytestmark = pytest.mark.gpu

V = s.VOCAB
WIDTHS = [32, 64, 96, 160, 928]
ROWS = [1, 3, 9, 66]


@pytest.fixture(scope="module")
def smp():
    b = s.BatchSampler(0)
    yield b
    b.close()


def make_head(cols: int, q8: bool, seed: int) -> np.ndarray:
    """A random head in promptboot's layout (vocab rows of 18- or 34-byte
    blocks with an fp16 scale first); a Q4_0 head of an odd block count gets
    one +inf scale in tile 7."""
    rng = np.random.default_rng(seed)
    blocks = cols // 32
    width = 34 if q8 else 18
    h = rng.integers(0, 256, (V, blocks, width), dtype=np.uint8)
    lo, hi = (0.0005, 0.004) if q8 else (0.001, 0.02)
    sc = rng.uniform(lo, hi, (V, blocks)).astype(np.float16).view(np.uint16)
    if not q8 and blocks % 2 == 1 and blocks > 1:
        sc[64 * 7 + 5, blocks - 1] = 0x7C00
    h[:, :, 0] = sc & 0xFF
    h[:, :, 1] = sc >> 8
    return h.reshape(-1)


@pytest.mark.parametrize("q8", [False, True], ids=["q4_0", "q8_0"])
@pytest.mark.parametrize("cols", WIDTHS)
def test_logits_and_draws_at_each_width(smp, q8, cols):
    import torch

    head = make_head(cols, q8, seed=cols + (1000 if q8 else 0))
    packed = smp.pack_lmhead(torch.from_numpy(head).to("cuda:0"), q8=q8, cols=cols)
    rng = np.random.default_rng(cols)
    for rows in ROWS:
        hidden = rng.standard_normal((rows, cols)).astype(np.float32)
        r24 = (np.arange(rows, dtype=np.uint32) * 7919 + 3) & 0xFFFFFF
        token = torch.empty(rows, dtype=torch.int32, device="cuda:0")
        logits = torch.empty((rows, V), dtype=torch.int32, device="cuda:0")
        smp.lmhead_sample(packed, to_dev(hidden), to_dev(r24), token=token, logits=logits,
                          cols=cols, q8=q8)
        torch.cuda.synchronize()
        glog = logits.cpu().numpy().view(np.uint32)
        rlog = o.lmhead_logits(hidden, head, V, cols, threads=16, q8=q8)
        gnan = np.isnan(glog.view(np.float32))
        rnan = np.isnan(rlog.view(np.float32))
        assert (gnan == rnan).all(), (cols, rows)
        bad = np.argwhere((glog != rlog) & ~rnan)
        assert bad.size == 0, (cols, rows, bad[:5])
        rtok, _, _, _ = o.sample_batch(rlog, np.zeros((rows, 1), np.uint32),
                                       np.zeros(rows, np.uint32), r24, threads=4)
        gtok = token.cpu().numpy().view(np.uint32)
        assert (gtok == rtok).all(), (cols, rows)
