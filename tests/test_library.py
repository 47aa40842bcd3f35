"""torch.library registration (CPU): the custom operators exist and their
fake implementations give the shapes and dtypes the kernels produce."""
import pytest
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


@pytest.mark.parametrize("d,dk", [(40, 40), (36, 40)])
def test_fake_shapes_general_inputs(d, dk):
    """float16 at d = 40 (whole 16-byte chunks: taken as is) and d = 36
    (padded to 40): the operator's output is in the kernels' layout, the
    input dtype; the gradients in the caller's."""
    Q = torch.empty(1, 2, 70, d, device="meta", dtype=torch.float16)
    outs = torch.ops.adasplash.forward(Q, Q, Q, None, None, 1.5, 8, d ** -0.5, "entmax")
    assert (tuple(outs[0].shape), outs[0].dtype) == ((1, 2, 70, dk), torch.float16)
    g = torch.ops.adasplash.backward(Q, Q, Q, None, None, outs[0], outs[0], *outs[1:], 1.5, 8,
                                     d ** -0.5, "entmax")
    assert [(tuple(x.shape), x.dtype) for x in g] == [((1, 2, 70, d), torch.float16)] * 3


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
    assert args.bwd_passes == "support"
    assert benchmark.build_parser().parse_args(["--bwd-passes", "tiles"]).bwd_passes == "tiles"
    with pytest.raises(SystemExit):
        benchmark.build_parser().parse_args(["--bwd-passes", "dense"])


def test_benchmark_cli_rocprof_command_and_summary(tmp_path):
    """--rocprof-pmc: the child command puts the interpreter right after
    "--" (rocprofv3 must start the program itself) and drops the rocprof
    options; the summary averages each library kernel's counters over its
    dispatches and ignores other kernels."""
    import sys

    from splash_attention import benchmark

    argv = ["--config", "1x2x256x64", "--rocprof-pmc", "SQ_WAVES SQ_INSTS_VALU",
            "--rocprof-dir=/x", "--backward"]
    cmd = benchmark.rocprof_command(argv, "SQ_WAVES SQ_INSTS_VALU", "/out")
    assert cmd[:4] == ["rocprofv3", "--pmc", "SQ_WAVES", "SQ_INSTS_VALU"]
    i = cmd.index("--")
    assert cmd[i + 1:i + 4] == [sys.executable, "-m", "splash_attention.benchmark"]
    assert cmd[i + 4:] == ["--config", "1x2x256x64", "--backward"]
    assert cmd[cmd.index("-d") + 1] == "/out"
    (tmp_path / "host" / "1").mkdir(parents=True)
    rows = [
        ("void asa::(anonymous namespace)::select_kernel<unsigned short, 64, 0, 2>(asa::SelectParams)",
         "SQ_WAVES", 16384.0),
        ("void asa::(anonymous namespace)::select_kernel<unsigned short, 64, 0, 2>(asa::SelectParams)",
         "SQ_WAVES", 8192.0),
        ("void asa::(anonymous namespace)::tau_kernel(asa::SelectParams)", "SQ_WAVES", 64.0),
        ("void at::native::elementwise_kernel<128, 4>(int)", "SQ_WAVES", 7.0),
    ]
    with open(tmp_path / "host" / "1" / "run_counter_collection.csv", "w") as f:
        f.write('"Dispatch_Id","Kernel_Name","Counter_Name","Counter_Value"\n')
        for n, (k, c, v) in enumerate(rows):
            f.write(f'{n},"{k}","{c}",{v}\n')
    s = benchmark.pmc_summary(str(tmp_path))
    assert s == {"select_kernel": {"SQ_WAVES": 12288.0}, "tau_kernel": {"SQ_WAVES": 64.0}}
