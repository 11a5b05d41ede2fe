"""thq_weight_from_gguf on the GPU: tensors of a GGUF file (written by
tests/gguf_writer.py) become weights whose block bytes, dequantization and
matmul match the oracle. This is the loader's path from Content::tensor to
QMatMul (engine/src/model.rs:526-562, ModelWeights::from_gguf).
"""
import numpy as np
import pytest
import torch

import gguf_writer as G
import oracle as O
from helpers import activations, q6k_bytes, rel_row_err, weight_bytes

pytestmark = pytest.mark.gpu

thq = pytest.importorskip("thq")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.init()
    yield
    torch.cuda.synchronize()


def test_weights_from_a_gguf_file(tmp_path):
    q4 = weight_bytes(O.Q4_K, 96, 1024, seed=21)
    q8 = weight_bytes(O.Q8_0, 40, 512, seed=22)
    q6 = q6k_bytes(72, 2048, seed=23)
    tensors = [
        ("blk.0.ffn_gate.weight", O.Q4_K, (96, 1024), q4.tobytes()),
        ("blk.0.attn_q.weight", O.Q8_0, (40, 512), q8.tobytes()),
        ("output.weight", O.Q6_K, (72, 2048), q6.tobytes()),
        ("output_norm.weight", 0, (2048,), np.ones(2048, np.float32).tobytes()),
        ("blk.0.attn_q.bias1d", O.Q8_0, (64,), q8[0, :68].tobytes()),
    ]
    kv = [("general.architecture", G.STRING, "qwen3"), ("general.alignment", G.U32, 64)]
    data, _, _ = G.build(kv, tensors)
    path = tmp_path / "w.gguf"
    path.write_bytes(data)
    with thq.GGUFFile(str(path)) as f:
        for name, qt, (n, k), blob in tensors[:3]:
            w = f.weight(name)
            assert w.dtype == qt and w.shape == (n, k)
            raw = np.frombuffer(blob, np.uint8).reshape(n, -1)
            assert np.array_equal(w.data(), raw)
            want = O.dequantize(qt, raw, n, k)
            assert np.array_equal(w.dequantize().cpu().numpy().view(np.uint32), want.view(np.uint32))
            x = O.bf16_round(activations(3, k, seed=24))
            y = thq.matmul(w, torch.from_numpy(x).cuda().to(torch.bfloat16), torch.float32).cpu().numpy()
            assert rel_row_err(y, O.matmul(qt, raw, n, k, x)) <= 1e-2
            x1 = O.bf16_round(activations(1, k, seed=25))
            y1 = thq.matmul(w, torch.from_numpy(x1).cuda().to(torch.bfloat16), torch.float32).cpu().numpy()
            assert rel_row_err(y1, O.matmul(qt, raw, n, k, x1)) <= 1e-4
        with pytest.raises(thq.ThqError) as e:
            f.weight("output_norm.weight")
        assert e.value.code == thq.EDTYPE
        with pytest.raises(thq.ThqError) as e:
            f.weight("blk.0.attn_q.bias1d")
        assert e.value.code == thq.ESHAPE
        with pytest.raises(thq.ThqError) as e:
            f.weight("missing.weight")
        assert e.value.code == thq.ENOTFOUND
