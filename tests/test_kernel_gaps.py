"""tests/native/kernel_gaps.py (the serving loop's kernel-trace timeline)
on a hand-made trace: the loop's window, busy time and per-pair gaps."""
from __future__ import annotations

import importlib.util
import pathlib

SPEC = importlib.util.spec_from_file_location(
    "kernel_gaps", pathlib.Path(__file__).resolve().parent / "native" / "kernel_gaps.py")
kg = importlib.util.module_from_spec(SPEC)
SPEC.loader.exec_module(kg)


def test_window_busy_and_gaps():
    k = [
        (0, 10, "void dsdk::TableReserveKernel(int)"),            # before the loop
        (100, 110, "void dsdk::StageInKernel(dsdk::StageSegments)"),
        (110, 150, "void dsdk::(anonymous namespace)::FusedStepKernel<false>(int)"),
        (160, 170, "void dsdk::TablePlanAppendKernel(int)"),
        (170, 180, "void dsdk::StageInKernel(dsdk::StageSegments)"),
        (190, 230, "void dsdk::(anonymous namespace)::FusedStepKernel<false>(int)"),
        (300, 310, "__amd_rocclr_fillBufferAligned"),                # the next run
    ]
    w = kg.loop_window(k)
    assert [kg.short(n) for _, _, n in w] == ["StageInKernel", "FusedStepKernel",
                                              "TablePlanAppendKernel", "StageInKernel",
                                              "FusedStepKernel"]
    lines = kg.summarize(w)
    assert lines[0].startswith("kernels 5 window 0.000 ms busy 0.000 ms (0.85)")
    gap = next(x for x in lines if "StageInKernel" in x and "-> FusedStepKernel" in x)
    assert "n=    2" in gap and "mean    0.01" in gap  # gaps 0 and 10 ns
