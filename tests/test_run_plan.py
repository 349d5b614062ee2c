"""The MLIR-free planner (libnova_run) on CPU: programs written in the op
surface parse, get the launch plan the lowering would emit (folds of
widening casts and transposes into GEMM operands, of GELU and narrowing
casts into the epilogue, zero fills elided), infer the reference's result
types, and ops outside this path are refused by name."""
import os

import pytest

import nova_run
from conftest import GOLDEN

MLIR = os.path.join(GOLDEN, "mlir")


def prog(name):
    with open(os.path.join(MLIR, name)) as f:
        return nova_run.Program(f.read())


def test_linear_gelu_folds_into_one_gemm():
    p = prog("linear_gelu_bf16.mlir")
    plan = p.plan("linear_gelu")
    launches = [l for l in plan.splitlines() if "_mlir_ciface_" in l]
    assert len(launches) == 1
    assert "nova.linear + nova.gelu + nova.cast -> _mlir_ciface_nova_hip_gemm" in launches[0]
    assert "epilogue=bias+gelu" in launches[0]
    assert "strides(1,160)" in launches[0]          # the transposed weight is a view
    assert "bf16" in launches[0].split("->")[-1]    # bf16 output
    assert p.args("linear_gelu") == [(1, (96, 160)), (1, (200, 160)), (1, (200,))]
    assert p.results("linear_gelu") == [(1, (96, 200))]


def test_batch_matmul_forms():
    p = prog("batch_matmul_bf16.mlir")
    for f in ("bmm", "bmm_nova"):
        plan = p.plan(f)
        assert plan.count("_mlir_ciface_nova_hip_gemm") == 1
        assert "hipMemsetAsync" not in plan         # the zero fill only feeds the GEMM's outs
        assert p.results(f) == [(0, (4, 128, 160))]


def test_reductions_and_backward_plans():
    p = prog("reductions.mlir")
    assert p.results("ln") == [(0, (64, 1024)), (0, (64,)), (0, (64,))]
    assert "_mlir_ciface_nova_hip_layer_norm_backward_f32" in p.plan("ln_train")
    plan = p.plan("sce_train")
    # the softmax feeds only sce_backward: one fused launch
    assert "_mlir_ciface_nova_hip_sce_fwd_bwd_f32" in plan
    assert "_mlir_ciface_nova_hip_sce_backward_f32" not in plan
    assert p.results("sce_train") == [(0, (1,)), (0, (32, 5000))]
    b = prog("backward.mlir")
    assert b.results("lin_bwd") == [(0, (40, 36)), (0, (36, 24)), (0, (24,))]
    assert b.results("mm_bwd") == [(0, (64, 128)), (0, (128, 96))]


def test_memref_entry_writes_output_argument():
    p = prog("memref_main.mlir")
    plan = p.plan("main")
    assert "materialize_in_destination" in plan
    assert p.results("main") == []
    assert len(p.args("main")) == 4


def test_nova_matmul_bf16_infers_f16_result():
    """NovaOps.cpp:1198: bf16 x bf16 nova.matmul gives f16 (the planner then
    refuses it: its bf16 -> f16 accumulation is not on this path)."""
    p = nova_run.Program("""func.func @m(%a: tensor<8x16xbf16>, %b: tensor<16x4xbf16>) -> tensor<8x4xf16> {
      %r = nova.matmul %a, %b : tensor<8x16xbf16>, tensor<16x4xbf16>
      return %r : tensor<8x4xf16>
    }""")
    with pytest.raises(nova_run.NovaRunError, match="a 16-bit GEMM result accumulates in its own type"):
        p.plan("m")


def test_ops_outside_the_path_are_refused():
    with pytest.raises(nova_run.NovaRunError, match="nova.relu"):
        prog("not_on_path.mlir")
    p = nova_run.Program("""func.func @g(%x: tensor<4x8xf32>) -> tensor<4x8xf32> {
      %g = nova.gelu %x : tensor<4x8xf32>
      return %g : tensor<4x8xf32>
    }""")
    # a nova.gelu that cannot fold into a GEMM epilogue is its own kernel
    assert "nova.gelu -> _mlir_ciface_nova_hip_gelu_f32" in p.plan("g")
    p = nova_run.Program("""func.func @c(%x: tensor<4x8xf32>) -> tensor<4x8xbf16> {
      %c = nova.cast %x : tensor<4x8xf32> -> tensor<4x8xbf16>
      return %c : tensor<4x8xbf16>
    }""")
    with pytest.raises(nova_run.NovaRunError, match="not foldable"):
        p.plan("c")
    with pytest.raises(nova_run.NovaRunError, match="no function"):
        p.plan("missing")


def test_bad_syntax_and_types_are_reported_with_lines():
    with pytest.raises(nova_run.NovaRunError, match="line 2"):
        nova_run.Program("""func.func @f(%x: tensor<4x8xf32>) -> tensor<4x8xf32> {
          %r = nova.linear %x, %x : tensor<4x8xf32>
          return %r : tensor<4x8xf32>
        }""")
    with pytest.raises(nova_run.NovaRunError, match="unsupported"):
        nova_run.Program("func.func @f(%x: tensor<?x8xf32>) { return }")
    # sizes whose element or byte counts would overflow 64-bit products
    for t in ("99999999999999999999x8xf32", "1099511627777x8xf32",
              "1048576x1048576x1048576xf32", "0x8xf32x"):
        with pytest.raises(nova_run.NovaRunError, match="unsupported"):
            nova_run.Program("func.func @f(%x: tensor<" + t + ">) { return }")


def test_library_exports_every_declared_symbol():
    import re
    from conftest import REPO
    text = open(os.path.join(REPO, "include", "nova_run.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = sorted(set(re.findall(r"\b(nova_run_\w+)\s*\(", text)))
    assert len(names) >= 10
    L = nova_run.lib()
    for n in names:
        assert hasattr(L, n), n


def test_gpt_step_plans_every_op():
    from gpt_program import gpt_step
    p = nova_run.Program(gpt_step(2, 8, 64, 32, 64))
    plan = p.plan("gpt_step")
    for want in ("nova.gather -> _mlir_ciface_nova_hip_gather_f32",
                 "nova.add -> _mlir_ciface_nova_hip_binary_f32",
                 "nova.gelu -> _mlir_ciface_nova_hip_gelu_f32",
                 "i16 labels -> _mlir_ciface_nova_hip_index_to_i32",
                 "nova.constant splat 1 -> elided",
                 "nova.mul by splat 1.0 -> view",
                 "nova.gelu_backward -> _mlir_ciface_nova_hip_gelu_backward_f32",
                 "nova.reduce<sum> -> _mlir_ciface_nova_hip_reduce_sum_f32(",
                 "[2,8,32]f32 as [1,2,256])",
                 "nova.scatter_add -> _mlir_ciface_nova_hip_scatter_add_f32",
                 "nova.reshape -> view b0[16]i16"):
        assert want in plan, want
    # the linear whose output feeds gelu and gelu_backward keeps its own GELU
    assert "epilogue=bias+gelu" not in plan
    assert plan.count("_mlir_ciface_nova_hip_gemm") == 5
    assert p.args("gpt_step")[0] == (5, (2, 8))
    assert p.results("gpt_step")[0] == (0, (1,)) and p.results("gpt_step")[1] == (0, (64, 32))


@pytest.mark.parametrize("body,msg", [
    ("%r = nova.reduce<max> %x dimension = [0] : tensor<4x8xf32>", "only the sum reduction"),
    ("%r = nova.constant {value = dense<[1.0, 2.0]> : tensor<2xf32>} : tensor<2xf32>", "splat"),
    ("%r = nova.gather %x [%i] {axis = 1} : tensor<4x8xf32>, tensor<3xi32> -> tensor<4x3xf32>",
     "axis 0 only"),
])
def test_glue_forms_outside_the_path_are_refused(body, msg):
    text = ("func.func @f(%x: tensor<4x8xf32>, %i: tensor<3xi32>) -> tensor<4x8xf32> {\n  "
            + body + "\n  return %x : tensor<4x8xf32>\n}\n")
    p = nova_run.Program(text)
    with pytest.raises(nova_run.NovaRunError, match=msg):
        p.plan("f")


def _gemm_outputs(plan):
    """Output buffer id of each GEMM launch in a plan text."""
    import re
    outs = []
    for line in plan.splitlines():
        if "_mlir_ciface_nova_hip_gemm(" in line:
            outs.append(int(re.search(r"\) -> b(\d+)\[", line).group(1)))
    return outs


def test_gemms_over_one_cse_fill_get_their_own_buffers():
    """After CSE (Pipeline.cpp:86) two products may share one zero fill; each
    result is a new tensor, so they must not land in one buffer."""
    p = nova_run.Program("""func.func @two(%a: tensor<8x16xf32>, %b: tensor<16x4xf32>, %c: tensor<16x4xf32>) -> (tensor<8x4xf32>, tensor<8x4xf32>) {
      %z = arith.constant 0.000000e+00 : f32
      %e = tensor.empty() : tensor<8x4xf32>
      %f = linalg.fill ins(%z : f32) outs(%e : tensor<8x4xf32>) -> tensor<8x4xf32>
      %r1 = linalg.matmul ins(%a, %b : tensor<8x16xf32>, tensor<16x4xf32>) outs(%f : tensor<8x4xf32>) -> tensor<8x4xf32>
      %r2 = linalg.matmul ins(%a, %c : tensor<8x16xf32>, tensor<16x4xf32>) outs(%f : tensor<8x4xf32>) -> tensor<8x4xf32>
      return %r1, %r2 : tensor<8x4xf32>, tensor<8x4xf32>
    }""")
    outs = _gemm_outputs(p.plan("two"))
    assert len(outs) == 2 and outs[0] != outs[1]
    assert "hipMemsetAsync" not in p.plan("two")


def test_fill_into_an_argument_leaves_the_argument_alone():
    """linalg.fill outs(%x) makes a new tensor: %x keeps its values for the
    second product, which reads it."""
    p = nova_run.Program("""func.func @f(%a: tensor<8x8xf32>, %x: tensor<8x8xf32>) -> (tensor<8x8xf32>, tensor<8x8xf32>) {
      %z = arith.constant 0.000000e+00 : f32
      %f = linalg.fill ins(%z : f32) outs(%x : tensor<8x8xf32>) -> tensor<8x8xf32>
      %r1 = linalg.matmul ins(%a, %a : tensor<8x8xf32>, tensor<8x8xf32>) outs(%f : tensor<8x8xf32>) -> tensor<8x8xf32>
      %r2 = nova.matmul %x, %a : tensor<8x8xf32>, tensor<8x8xf32>
      return %r1, %r2 : tensor<8x8xf32>, tensor<8x8xf32>
    }""")
    outs = _gemm_outputs(p.plan("f"))
    assert len(outs) == 2 and 1 not in outs and outs[0] != outs[1]   # b1 is %x


def test_sole_fill_user_writes_the_empty_buffer_in_place():
    p = prog("batch_matmul_bf16.mlir")
    plan = p.plan("bmm")
    assert _gemm_outputs(plan) == [2]     # b0, b1 arguments; b2 the tensor.empty


def test_narrow_accumulators():
    """An f16 x f16 nova.matmul (result f16, NovaOps.cpp:1198) and a linalg
    matmul with bf16 ins and outs accumulate in the narrow type; a bf16 x
    bf16 nova.matmul (f16 result through a bf16 -> f16 cast) is refused."""
    p = nova_run.Program("""func.func @h(%a: tensor<8x16xf16>, %b: tensor<16x4xf16>) -> tensor<8x4xf16> {
      %r = nova.matmul %a, %b : tensor<8x16xf16>, tensor<16x4xf16>
      return %r : tensor<8x4xf16>
    }
    func.func @l(%a: tensor<8x16xbf16>, %b: tensor<16x4xbf16>) -> tensor<8x4xbf16> {
      %z = arith.constant 0.000000e+00 : bf16
      %e = tensor.empty() : tensor<8x4xbf16>
      %f = linalg.fill ins(%z : bf16) outs(%e : tensor<8x4xbf16>) -> tensor<8x4xbf16>
      %r = linalg.matmul ins(%a, %b : tensor<8x16xbf16>, tensor<16x4xbf16>) outs(%f : tensor<8x4xbf16>) -> tensor<8x4xbf16>
      return %r : tensor<8x4xbf16>
    }
    func.func @lin(%x: tensor<8x16xf16>, %w: tensor<16x4xf16>, %b: tensor<4xf16>) -> tensor<8x4xf16> {
      %y = nova.linear %x, %w, %b : tensor<8x16xf16>, tensor<16x4xf16>, tensor<4xf16>
      return %y : tensor<8x4xf16>
    }
    func.func @m(%a: tensor<8x16xbf16>, %b: tensor<16x4xbf16>) -> tensor<8x4xf16> {
      %r = nova.matmul %a, %b : tensor<8x16xbf16>, tensor<16x4xbf16>
      return %r : tensor<8x4xf16>
    }""")
    assert "accumulate=f16" in p.plan("h")
    assert "accumulate=bf16" in p.plan("l")
    assert "accumulate=f16" in p.plan("lin") and "epilogue=bias" in p.plan("lin")
    with pytest.raises(nova_run.NovaRunError, match="a 16-bit GEMM result accumulates in its own type"):
        p.plan("m")
    # the f32-accumulate forms are unchanged
    b = prog("batch_matmul_bf16.mlir")
    assert "accumulate=" not in b.plan("bmm") and "accumulate=" not in b.plan("bmm_nova")


def test_gpt_step_fused_sce_and_elided_unit_multiply():
    """nova.sce whose softmax feeds only nova.sce_backward over the same labels
    is one fused launch (no softmax written); the multiply by a splat 1.0 and
    its fill disappear."""
    from gpt_program import gpt_step
    plan = nova_run.Program(gpt_step(2, 8, 64, 32, 64)).plan("gpt_step")
    assert "_mlir_ciface_nova_hip_sce_fwd_bwd_f32" in plan
    assert "_mlir_ciface_nova_hip_sce_f32(" not in plan
    assert "_mlir_ciface_nova_hip_sce_backward_f32" not in plan
    assert "splat 1 -> elided" in plan and "nova.mul by splat 1.0 -> view" in plan
    assert "nova.constant splat 1 -> _mlir_ciface_nova_hip_fill_f32" not in plan
    assert plan.count("i16 labels -> _mlir_ciface_nova_hip_index_to_i32") == 1


def test_unit_multiply_kept_when_it_broadcasts_or_escapes():
    p = nova_run.Program("""func.func @b(%x: tensor<4x1xf32>) -> tensor<4x8xf32> {
      %one = nova.constant {value = dense<1.000000e+00> : tensor<4x8xf32>} : tensor<4x8xf32>
      %y = nova.mul %x, %one : tensor<4x1xf32>, tensor<4x8xf32>
      return %y : tensor<4x8xf32>
    }
    func.func @r(%x: tensor<4x8xf32>) -> (tensor<4x8xf32>, tensor<1xf32>) {
      %one = nova.constant {value = dense<1.000000e+00> : tensor<1xf32>} : tensor<1xf32>
      %y = nova.mul %x, %one : tensor<4x8xf32>, tensor<1xf32>
      return %y, %one : tensor<4x8xf32>, tensor<1xf32>
    }
    func.func @s(%x: tensor<8x5xf32>, %t: tensor<8xi32>) -> (tensor<8x5xf32>, tensor<1xf32>, tensor<8x5xf32>) {
      %sce:2 = nova.sce %x, %t : tensor<8x5xf32>, tensor<8xi32>
      %g = nova.sce_backward %sce#0, %t : tensor<8x5xf32>, tensor<8xi32>
      return %sce#0, %sce#1, %g : tensor<8x5xf32>, tensor<1xf32>, tensor<8x5xf32>
    }""")
    assert "_mlir_ciface_nova_hip_binary_f32" in p.plan("b")    # broadcasting: a real multiply
    assert "_mlir_ciface_nova_hip_binary_f32" in p.plan("r")    # the constant is returned
    plan = p.plan("s")                                          # softmax also returned: no fold
    assert "_mlir_ciface_nova_hip_sce_f32" in plan and "sce_backward_f32" in plan


def test_f32_gemm_mode_marks_every_f32_product():
    from gpt_program import gpt_step
    p = nova_run.Program(gpt_step(2, 8, 64, 32, 64))
    assert "f32=mfma" not in p.plan("gpt_step")
    p.set_f32_gemm(nova_run.F32_GEMM_MFMA)
    plan = p.plan("gpt_step")
    gemm_lines = [l for l in plan.splitlines() if "_mlir_ciface_nova_hip_gemm(" in l
                  or "_backward(" in l and ("linear_backward" in l or "matmul_backward" in l)]
    assert gemm_lines and all("f32=mfma" in l for l in gemm_lines)
    p.set_f32_gemm(nova_run.F32_GEMM_EXACT)
    assert "f32=mfma" not in p.plan("gpt_step")
    with pytest.raises(nova_run.NovaRunError, match="mode"):
        p.set_f32_gemm(7)


def test_rank4_matmul_plans_and_batch_transpose_is_refused():
    """nova.matmul above rank 3 folds its batch dims into one launch; a
    transpose of batch axes leaves leading dims the launch cannot fold and
    is refused at plan time instead of being addressed wrongly, as are SCE
    labels given as a transposed view."""
    p = prog("matmul_rank4.mlir")
    for f in ("mm4", "mm4_bcast"):
        assert p.plan(f).count("_mlir_ciface_nova_hip_gemm") == 1
        assert p.results(f) == [(0, (2, 3, 8, 5))]
    with pytest.raises(nova_run.NovaRunError, match="leading dims are not contiguous"):
        p.plan("mm4_batch_transposed")
    with pytest.raises(nova_run.NovaRunError, match="operand 1 is a view whose leading dims"):
        p.plan("sce_labels_transposed")


ACC_PROGRAMS = """func.func @arg(%A: tensor<256x128xf32>, %B: tensor<128x512xf32>, %C: tensor<256x512xf32>) -> tensor<256x512xf32> {
  %r = linalg.matmul ins(%A, %B : tensor<256x128xf32>, tensor<128x512xf32>) outs(%C : tensor<256x512xf32>) -> tensor<256x512xf32>
  return %r : tensor<256x512xf32>
}
func.func @chain(%A: tensor<8x16xf32>, %B: tensor<16x4xf32>, %D: tensor<8x4xf32>, %E: tensor<4x4xf32>) -> tensor<8x4xf32> {
  %p = nova.matmul %A, %B : tensor<8x16xf32>, tensor<16x4xf32>
  %r = linalg.matmul ins(%D, %E : tensor<8x4xf32>, tensor<4x4xf32>) outs(%p : tensor<8x4xf32>) -> tensor<8x4xf32>
  return %r : tensor<8x4xf32>
}
func.func @reread(%A: tensor<8x16xf32>, %B: tensor<16x4xf32>, %D: tensor<8x4xf32>, %E: tensor<4x4xf32>) -> (tensor<8x4xf32>, tensor<8x4xf32>) {
  %p = nova.matmul %A, %B : tensor<8x16xf32>, tensor<16x4xf32>
  %r = linalg.matmul ins(%D, %E : tensor<8x4xf32>, tensor<4x4xf32>) outs(%p : tensor<8x4xf32>) -> tensor<8x4xf32>
  return %r, %p : tensor<8x4xf32>, tensor<8x4xf32>
}
func.func @batch(%A: tensor<4x64x256xf32>, %B: tensor<4x256x64xf32>, %C: tensor<4x64x64xf32>) -> tensor<4x64x64xf32> {
  %r = linalg.batch_matmul ins(%A, %B : tensor<4x64x256xf32>, tensor<4x256x64xf32>) outs(%C : tensor<4x64x64xf32>) -> tensor<4x64x64xf32>
  return %r : tensor<4x64x64xf32>
}
func.func @narrow(%A: tensor<8x16xf16>, %B: tensor<16x4xf16>, %C: tensor<8x4xf16>) -> tensor<8x4xf16> {
  %r = linalg.matmul ins(%A, %B : tensor<8x16xf16>, tensor<16x4xf16>) outs(%C : tensor<8x4xf16>) -> tensor<8x4xf16>
  return %r : tensor<8x4xf16>
}
func.func @wide16(%A: tensor<8x16xbf16>, %B: tensor<16x4xbf16>, %C: tensor<8x4xf32>) -> tensor<8x4xf32> {
  %r = linalg.matmul ins(%A, %B : tensor<8x16xbf16>, tensor<16x4xbf16>) outs(%C : tensor<8x4xf32>) -> tensor<8x4xf32>
  return %r : tensor<8x4xf32>
}
func.func @uninit(%A: tensor<8x16xf32>, %B: tensor<16x4xf32>) -> tensor<8x4xf32> {
  %e = tensor.empty() : tensor<8x4xf32>
  %r = linalg.matmul ins(%A, %B : tensor<8x16xf32>, tensor<16x4xf32>) outs(%e : tensor<8x4xf32>) -> tensor<8x4xf32>
  return %r : tensor<8x4xf32>
}
"""


def test_linalg_matmul_accumulates_into_data_holding_outs():
    """linalg.matmul outs(%C) with %C holding data (the reference's
    pipeline-test form, 02_matmul_aligned.mlir:15-19): one exact GEMM that
    sums from C's values.  A function argument keeps its data (the sums go
    into a copy); a sole-use intermediate is summed into in place; an
    intermediate that is read again is copied first."""
    p = nova_run.Program(ACC_PROGRAMS)
    plan = p.plan("arg")
    assert plan.count("hipMemcpyAsync") == 1 and "accumulate-into=f32" in plan
    assert 2 not in _gemm_outputs(plan)                       # b2 is %C
    assert p.results("arg") == [(0, (256, 512))]
    chain = p.plan("chain")
    assert "hipMemcpyAsync" not in chain
    outs = _gemm_outputs(chain)
    assert len(outs) == 2 and outs[0] == outs[1]              # in place
    reread = p.plan("reread")
    assert reread.count("hipMemcpyAsync") == 1
    outs = _gemm_outputs(reread)
    assert len(outs) == 2 and outs[0] != outs[1]
    assert "accumulate-into=f32" in p.plan("batch")
    narrow = p.plan("narrow")
    assert "accumulate-into=f16" in narrow
    # f32 matrix-core mode leaves the accumulate form on the exact kernel
    p.set_f32_gemm(nova_run.F32_GEMM_MFMA)
    assert "f32=mfma" not in p.plan("arg")
    assert "f32=mfma" in p.plan("chain")   # the plain nova.matmul in front of it
    p.set_f32_gemm(nova_run.F32_GEMM_EXACT)


def test_linalg_matmul_accumulate_forms_off_the_path():
    p = nova_run.Program(ACC_PROGRAMS)
    with pytest.raises(nova_run.NovaRunError, match="16-bit operands accumulating into data-holding"):
        p.plan("wide16")
    with pytest.raises(nova_run.NovaRunError, match="uninitialised tensor.empty"):
        p.plan("uninit")
