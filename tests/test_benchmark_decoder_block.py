"""The decoder-block benchmark's model and argument checks on the CPU (the
timed run needs a GPU and is covered by the gpu-marked test)."""
import pytest
import torch

from kotflash_amd import benchmark_decoder_block as bdb


def test_block_backends_agree_on_cpu():
    torch.manual_seed(0)
    block = bdb.DecoderBlock(4, 2, 16, attention_dtype=torch.float32)
    x = torch.randn(2, 24, 64)
    a = block(x, "sdpa_expanded_kv")
    b = block(x, "sdpa_native_gqa")
    assert a.shape == x.shape
    assert torch.allclose(a, b, atol=1e-5, rtol=1e-5)
    with pytest.raises(ValueError, match="unknown attention backend"):
        block(x, "nope")


@pytest.mark.parametrize("argv, message", [
    (["--q-heads", "6", "--kv-heads", "4"], "divisible"),
    (["--iterations", "2"], "three measured iterations"),
    (["--warmup", "0"], "at least one warmup"),
    (["--seq", "0"], "must be positive"),
])
def test_argument_checks(argv, message, capsys):
    with pytest.raises(SystemExit):
        bdb.parse_args(argv)
    assert message in capsys.readouterr().err
