"""The generic UOp-block renderer on a host without a GPU: each example
schedule's blocks render to HIP C++ and compile with hiprtc for gfx950
(dgen_hip_render_blocks), the Python UOp vocabulary matches the C ABI's
enums, and malformed blocks fail with a status and a message."""
import os
import re

import pytest

from dgen_hip import OscBankConfig
from dgen_hip import runtime as R
from dgen_hip import uop as U
from dgen_hip.uop_programs import (expr_uop_program, hop_uop_program, noise_uop_program, oscbank_uop_program,
                                   table_uop_program)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = open(os.path.join(ROOT, "include", "dgen_hip.h")).read()


def test_uop_vocabulary_matches_the_header():
    body = HEADER[HEADER.index("enum dgen_hip_uop_op {"):]
    body = body[:body.index("};")]
    names = re.findall(r"DGEN_HIP_UOP_(\w+)", body)
    camel = [n.lower() for n in U.OP_NAMES]
    assert [n.lower().replace("_", "") for n in names] == [c.replace("_", "") for c in camel]
    disp = dict((k, int(v)) for k, v in re.findall(r"DGEN_HIP_DISPATCH_(\w+) = (\d+)", HEADER))
    assert sorted(disp.values()) == sorted(U.DISPATCH.values())
    assert R.K_UOP_BLOCK == int(re.search(r"DGEN_HIP_K_UOP_BLOCK = (\d+)", HEADER).group(1))


@pytest.mark.parametrize("build", [
    lambda: oscbank_uop_program(OscBankConfig(frames=4096)),
    lambda: oscbank_uop_program(OscBankConfig(frames=4096), drive=2.0),
    lambda: hop_uop_program(4096, 256),
    lambda: noise_uop_program(1024),
    lambda: expr_uop_program(1024),
    lambda: table_uop_program(1024, 64),
], ids=["oscbank", "oscbank-shaper", "hop", "noise", "expr", "static-table"])
def test_example_blocks_render_and_compile(build):
    p = build()
    src = U.render(p.blocks, compile=True)
    assert src.count("extern \"C\" __global__ void dgen_block_") == len(p.blocks)
    for i, b in enumerate(p.blocks):
        assert f"dgen_block_{i}(" in src


def test_renderer_wraps_each_dispatch_mode_as_the_metal_renderer_does():
    p = hop_uop_program(4096, 256)
    src = U.render(p.blocks)
    k0 = src[src.index("dgen_block_0"):src.index("dgen_block_1")]
    k1 = src[src.index("dgen_block_1"):]
    # singleThreaded: one thread looping over the frames
    assert "if (id < 1u) {" in k0 and "for (unsigned i = 0; i < frameCount; i += 1u) {" in k0
    # perFrame, hop-based: one thread per frame, the counter's tape value checked for 0
    assert "if (id < frameCount) {" in k1 and "== 0.0f) {" in k1
    # tape globals at slot * frameCount + frame; the static table's global at frame 0
    assert "t[DG_T((unsigned long long)1u * frameCount + i)]" in k0
    t = U.render(table_uop_program(1024, 64).blocks)
    assert "t[DG_T((unsigned long long)0u * frameCount + 0u)]" in t
    assert "const unsigned i = 0;" in t


def _one(op, **kw):
    blk = U.Block(dispatch="perFrame")
    b = U.BlockBuilder(blk)
    b.op(op, **kw)
    return blk


def test_malformed_blocks_fail_with_a_message():
    L = R.load_library()
    bad = [
        (U.Block(dispatch="perFrame", ops=[U.UOp("endLoop")]), "unbalanced"),
        (U.Block(dispatch="perFrame", ops=[U.UOp("beginLoop", a=U.const(4))]), "unbalanced"),
        (U.Block(dispatch="fixedWithFrameLoop", n=0), "fixedWithFrameLoop"),
        (U.Block(dispatch="perFrame", ops=[U.UOp("add", value=U.const(1), a=U.const(1), b=U.const(2))]),
         "non-variable"),
        (U.Block(dispatch="perFrame", ops=[U.UOp("store", a=U.const(1), imm=(-3, 0))]), "cell"),
    ]
    for blk, msg in bad:
        with pytest.raises(R.HIPError, match=msg):
            U.render([blk])
    # a block whose C++ does not compile: hiprtc's log comes back
    blk = U.Block(dispatch="perFrame", ops=[U.UOp("add", value=U.var(1), a=U.var(7), b=U.const(1))])
    with pytest.raises(R.HIPError, match="compile failed"):
        U.render([blk], compile=True)
    assert L.dgen_hip_set_blocks(None, None, 0) == -1
    with pytest.raises(ValueError, match="GEMM"):
        U.render([U.Block(dispatch="gemm")])
