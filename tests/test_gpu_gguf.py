"""GPU: a GGUF model file loaded into device memory (tlh_gguf_layout / upload)
holds the file's bytes exactly, and the decoder built from its metadata and
weights (tensorlisp_amd.gguf.decoder_config / decoder_weights) reproduces the
reference CPU backend's decoder steps (tests/golden/decoder.npz, the same
weights) -- the path of the reference's `--device native` model load
(crates/tensorlisp/src/native_cuda.rs:44-82)."""
from __future__ import annotations

import numpy as np
import pytest

from refs import DECODER_STEPS, decoder_tiny_config, decoder_weights
from tensorlisp_amd import gguf
from test_gpu_executor import GpuDecoder, check_steps, gold

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("alignment", [32, 64])
def test_upload_holds_the_files_bytes(gpu, tmp_path, alignment):
    import torch

    c = decoder_tiny_config()
    p = tmp_path / "tiny.gguf"
    gguf.write_llama(p, c, decoder_weights(c), alignment)
    g = gguf.GgufFile(p)
    buf, views = g.load()
    torch.cuda.synchronize()
    assert len(views) == len(g.tensors)
    for t in g.tensors:
        v = views[t["name"]]
        assert v.data_ptr() % 256 == 0
        np.testing.assert_array_equal(v.cpu().numpy().reshape(-1), g.read(t["name"]).reshape(-1))


def test_decoder_from_a_gguf_file(gpu, tmp_path):
    c = decoder_tiny_config()
    p = tmp_path / "tiny.gguf"
    gguf.write_llama(p, c, decoder_weights(c))
    g = gguf.GgufFile(p)
    c2 = gguf.decoder_config(g, n_ctx=c.n_ctx)
    _, views = g.load()
    dec = GpuDecoder(c2, gguf.decoder_weights(c2, views), on_device=True)
    res = [dec.step(s)[2:] for s in DECODER_STEPS]
    gd = gold()
    n = len(DECODER_STEPS)
    check_steps(res, [gd[f"logits{i}"] for i in range(n)], [gd[f"argmax{i}"] for i in range(n)],
                [gd[f"cache{i}"] for i in range(2 * c.n_layer)], dec)
