"""torch.library registration (CPU): the custom operators exist and their
fake implementations give the shapes and dtypes the kernels produce."""
import torch

import splash_attention  # noqa: F401  (registers adasplash::forward / ::backward)


def test_ops_registered():
    assert hasattr(torch.ops.adasplash, "forward")
    assert hasattr(torch.ops.adasplash, "backward")


def test_fake_shapes_on_meta_tensors():
    Q = torch.empty(2, 3, 200, 64, device="meta", dtype=torch.bfloat16)
    K = torch.empty(2, 3, 130, 64, device="meta", dtype=torch.bfloat16)
    outs = torch.ops.adasplash.forward(Q, K, K, None, None, 1.5, 8, 0.125, "entmax")
    shapes = [(tuple(o.shape), o.dtype) for o in outs]
    # support masks: 4 waves x 64 lanes x 16 bits per tile slot
    assert shapes == [((2, 3, 200, 64), torch.bfloat16), ((6, 200), torch.float32),
                      ((6, 200), torch.float32), ((6, 4, 3), torch.uint8), ((6, 5), torch.int32),
                      ((6, 12), torch.int32), ((6, 4), torch.int32), ((6, 12), torch.int32),
                      ((6, 12, 4, 64), torch.int16)]
    g = torch.ops.adasplash.backward(Q, K, K, None, None, outs[0], outs[0], *outs[1:], 1.5, 8,
                                     0.125, "entmax")
    assert [tuple(x.shape) for x in g] == [(2, 3, 200, 64), (2, 3, 130, 64), (2, 3, 130, 64)]


def test_fake_shapes_general_inputs():
    """d not in {64, 128} and float16: the operator's output is in the
    kernels' layout (d padded to 64, float32); the gradients in the caller's."""
    Q = torch.empty(1, 2, 70, 40, device="meta", dtype=torch.float16)
    outs = torch.ops.adasplash.forward(Q, Q, Q, None, None, 1.5, 8, 40 ** -0.5, "entmax")
    assert (tuple(outs[0].shape), outs[0].dtype) == ((1, 2, 70, 64), torch.float32)
    g = torch.ops.adasplash.backward(Q, Q, Q, None, None, outs[0], outs[0], *outs[1:], 1.5, 8,
                                     40 ** -0.5, "entmax")
    assert [(tuple(x.shape), x.dtype) for x in g] == [((1, 2, 70, 40), torch.float16)] * 3


def test_benchmark_cli_parsing():
    import argparse

    import pytest

    from splash_attention import benchmark

    assert benchmark.parse_config("1x4x2048x64") == (1, 4, 2048, 64)
    with pytest.raises(argparse.ArgumentTypeError):
        benchmark.parse_config("1x4x2048")
    args = benchmark.build_parser().parse_args(["--config", "2x2x256x64", "--baseline", "vanilla",
                                                "--backward", "--dtype", "bf16"])
    assert args.config == [(2, 2, 256, 64)] and args.baseline == "vanilla" and args.backward
    assert args.tau_mode == "reference"
    assert benchmark.build_parser().parse_args(["--tau-mode", "exact"]).tau_mode == "exact"
