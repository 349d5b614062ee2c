//===- NovaHipLowering.cpp - Nova ops -> calls into libnova_hip -----------===//
//
// UNCOMPILED PROTOTYPE.  This image has no MLIR, so this file has never been
// built; its tested counterpart is the MLIR-free planner
// (runtime/nova_run.cpp), which carries the same rewrite and which every GPU
// test runs.  Both decide which op forms they lower from one table,
// include/nova_forms.h (nova_forms::check), so they accept and decline the
// same forms.
//
// The lowering takes Nova's GPU matmul / reduction ops (and the program glue
// around them) off the IREE-derived LLVMGPU sequence
// (lib/Transforms/LLVMGPU/Passes.cpp:115-372: TileAndDistribute,
// PromoteMatmulOperands, PadOperands, vector distribution, multibuffering)
// and calls the hand-written gfx950 kernels of libnova_hip instead.  It runs
// on the Nova ops themselves, ahead of Nova -> Linalg (Passes.cpp:88-90), so
// the ops it rewrites never reach that sequence.  A form the table declines
// keeps the existing path; with strict=true the pass instead fails on it
// (that path emits NVPTX, which cannot run on AMD).
//
// Each rewritten op becomes, in tensor form:
//   %b_i  = bufferization.to_buffer %operand_i read_only   (a view: see below)
//   %out  = memref.alloc() : <result type as a buffer>
//   %rc   = func.call @nova_hip_<op>(%b_0, ..., %out, ...) : (...) -> i32
//   cf.assert (%rc == 0), "libnova_hip <op> failed"
//   %res  = bufferization.to_tensor %out restrict writable
// with @nova_hip_<op> declared `private` and `llvm.emit_c_interface`, so the
// LLVM lowering calls _mlir_ciface_nova_hip_<op>(StridedMemRefType<T,R>*...),
// the entry points include/nova_hip.h declares.  Every buffer is passed as a
// memref with dynamic sizes, strides and offset: the descriptor layout of
// the C interface, whatever the static type.  The memref.alloc results are
// what the reference pipeline's ConvertMemRefToGpu turns into device
// allocations (ConvertMemRefToGpu.cpp:37-63).
//
// Every lowering first reads its operands, its folds and the table's verdict,
// and checks that each callee it needs can be declared with the type it
// needs; only then does it create ops.  A declined op leaves the IR as it was.
//
// Views and folds (the planner's, one each):
//   * nova.transpose of the last two dims feeding a GEMM operand is a
//     memref.transpose view (strided), not a copy;
//   * a widening nova.cast (bf16 / f16 -> f32) feeding a GEMM operand or
//     bias is dropped: the kernel reads the narrow data and accumulates in
//     f32;
//   * nova.linear / nova.matmul followed by a nova.gelu that is the result's
//     only use, and then a narrowing nova.cast that is the only use, fold
//     into the GEMM's epilogue (bias -> GELU -> round to bf16 / f16);
//   * leading dims fold into the batch (GEMMs) or row dim (row ops) through
//     collapse_shape views of the dense buffers: rank > 3 nova.matmul as
//     NovaToLinalg.cpp:904-988 collapses them, rank-3 nova.linear_backward
//     (the reference GPT step's own form, ltest/test.mlir:40, 42) as
//     [B*M, .];
//   * nova.sce whose softmax feeds only a nova.sce_backward over the same
//     targets is one fused call, and the softmax is never materialised;
//   * non-i32 targets / indices are widened by nova_hip_index_to_i32_* first;
//   * a linalg.(batch_)matmul whose outs holds data (not a zero fill) sums
//     from a copy of that data (NOVA_HIP_GEMM_ACC_C, the exact kernel).
// f32 GEMMs run the exact kernel (bit-identical to the CPU pipeline) unless
// the pass option f32-gemm=mfma selects the f32 matrix cores.
//
// Built only where MLIR is available (CMakeLists.txt next to this file,
// find_package(MLIR)).
//===----------------------------------------------------------------------===//

#include "Compiler/Dialect/nova/NovaDialect.h"
#include "Compiler/Dialect/nova/NovaOps.h"

#include "mlir/Dialect/Arith/IR/Arith.h"
#include "mlir/Dialect/Bufferization/IR/Bufferization.h"
#include "mlir/Dialect/ControlFlow/IR/ControlFlowOps.h"
#include "mlir/Dialect/Func/IR/FuncOps.h"
#include "mlir/Dialect/LLVMIR/LLVMDialect.h"
#include "mlir/Dialect/Linalg/IR/Linalg.h"
#include "mlir/Dialect/MemRef/IR/MemRef.h"
#include "mlir/Dialect/Tensor/IR/Tensor.h"
#include "mlir/IR/AffineMap.h"
#include "mlir/IR/BuiltinOps.h"
#include "mlir/IR/PatternMatch.h"
#include "mlir/Pass/Pass.h"
#include "mlir/Pass/PassRegistry.h"
#include "llvm/ADT/SmallPtrSet.h"
#include "llvm/ADT/TypeSwitch.h"

#include "nova_forms.h"
#include "nova_hip.h"

using namespace mlir;

namespace mlir::nova {

namespace {

constexpr int64_t kDyn = ShapedType::kDynamic;

// dtype code of include/nova_hip.h for a float / index element type, or -1.
int dtypeCode(Type t) {
  if (t.isF32()) return NOVA_HIP_DT_F32;
  if (t.isBF16()) return NOVA_HIP_DT_BF16;
  if (t.isF16()) return NOVA_HIP_DT_F16;
  if (t.isInteger(32)) return NOVA_HIP_DT_I32;
  if (t.isInteger(64)) return NOVA_HIP_DT_I64;
  if (t.isInteger(16)) return NOVA_HIP_DT_I16;
  return -1;
}

// The memref type the C interface passes as StridedMemRefType<T, rank>.
MemRefType abiType(Type elem, int64_t rank) {
  SmallVector<int64_t> shape(rank, kDyn), strides(rank, kDyn);
  return MemRefType::get(shape, elem,
                         StridedLayoutAttr::get(elem.getContext(), kDyn, strides));
}

RankedTensorType staticTensor(Value v) {
  auto t = dyn_cast<RankedTensorType>(v.getType());
  return t && t.hasStaticShape() ? t : RankedTensorType();
}

Value singleUse(Value v) { return v.hasOneUse() ? v : Value(); }

// What a GEMM operand reads: the tensor holding the data (through a widening
// cast and a transpose of the last two dims), and whether it is transposed.
struct GemmOperand {
  Value tensor;
  bool transposed = false;
  Type stored;  // element type of the data read
};

bool widening(CastOp c) {
  Type from = getElementTypeOrSelf(c.getInput().getType());
  return getElementTypeOrSelf(c.getType()).isF32() && (from.isBF16() || from.isF16());
}

GemmOperand traceOperand(Value v) {
  GemmOperand o;
  o.tensor = v;
  if (auto c = v.getDefiningOp<CastOp>())
    if (widening(c)) o.tensor = c.getInput();
  if (auto t = o.tensor.getDefiningOp<TransposeOp>()) {
    auto ty = cast<RankedTensorType>(t.getInput().getType());
    const int64_t r = ty.getRank();
    int64_t a1 = t.getAxes1(), a2 = t.getAxes2();
    if (a1 < 0) a1 += r;
    if (a2 < 0) a2 += r;
    if (r >= 2 && ((a1 == r - 1 && a2 == r - 2) || (a1 == r - 2 && a2 == r - 1))) {
      o.tensor = t.getInput();
      o.transposed = true;
      if (auto c = o.tensor.getDefiningOp<CastOp>())
        if (widening(c)) o.tensor = c.getInput();
    }
  }
  o.stored = getElementTypeOrSelf(o.tensor.getType());
  return o;
}

// The operands of one op as nova_forms sees them.
struct Form {
  SmallVector<nova_forms::Operand, 5> ops;
  SmallVector<SmallVector<int64_t, 8>, 5> shapes;
  bool ok = true;  // every operand a static ranked tensor
  // `v` is the value the op reads (its shape and logical type); `stored` the
  // element type of the data behind it (through folded casts).
  void add(Value v, Type stored) {
    auto t = staticTensor(v);
    if (!t) {
      ok = false;
      return;
    }
    shapes.emplace_back(t.getShape().begin(), t.getShape().end());
    nova_forms::Operand o;
    o.stored = dtypeCode(stored);
    o.logical = dtypeCode(t.getElementType());
    o.rank = (int)t.getRank();
    ops.push_back(o);
  }
  void add(Value v) { add(v, getElementTypeOrSelf(v.getType())); }
};

class Lowerer {
 public:
  Lowerer(ModuleOp m, bool f32Mfma) : module(m), rewriter(m.getContext()), f32Mfma(f32Mfma) {}

  // Ops the table declined (for strict mode), with the reason.
  SmallVector<std::pair<Operation *, std::string>> declinedOps;

  // Asks the form table about `op` (named `name` there).  True, and the op
  // recorded with the reason, when the op is not on this path.
  bool declined(Operation *op, const char *name, Form &f, const nova_forms::Attrs &at = {}) {
    if (!f.ok) {
      declinedOps.push_back({op, "operands are not statically shaped ranked tensors"});
      return true;
    }
    for (size_t i = 0; i < f.ops.size(); ++i) f.ops[i].shape = f.shapes[i].data();
    SmallVector<int> res;
    for (Type t : op->getResultTypes()) res.push_back(dtypeCode(getElementTypeOrSelf(t)));
    const char *why = nova_forms::check(name, (int)f.ops.size(), f.ops.data(), (int)res.size(),
                                        res.data(), at);
    if (why) declinedOps.push_back({op, why});
    return why != nullptr;
  }

  // ---- building blocks (called only after every check has passed) --------

  // Dense buffer of a tensor value.
  Value dense(Location loc, Value tensor) {
    auto tt = cast<RankedTensorType>(tensor.getType());
    return rewriter.create<bufferization::ToBufferOp>(
        loc, MemRefType::get(tt.getShape(), tt.getElementType()), tensor, /*readOnly=*/true);
  }

  // A view of the dense buffer `b` (identity layout) with another static
  // shape of the same element count, row-major.
  Value reshaped(Location loc, Value b, ArrayRef<int64_t> shape) {
    auto mt = cast<MemRefType>(b.getType());
    SmallVector<int64_t> strides(shape.size(), 1);
    for (int64_t i = (int64_t)shape.size() - 2; i >= 0; --i) strides[i] = strides[i + 1] * shape[i + 1];
    auto layout = StridedLayoutAttr::get(rewriter.getContext(), 0, strides);
    auto t = MemRefType::get(shape, mt.getElementType(), layout);
    SmallVector<OpFoldResult> sz, st;
    for (int64_t d : shape) sz.push_back(rewriter.getIndexAttr(d));
    for (int64_t d : strides) st.push_back(rewriter.getIndexAttr(d));
    return rewriter.create<memref::ReinterpretCastOp>(loc, t, b, rewriter.getIndexAttr(0), sz, st);
  }

  Value toAbi(Location loc, Value b) {
    auto mt = cast<MemRefType>(b.getType());
    return rewriter.create<memref::CastOp>(loc, abiType(mt.getElementType(), mt.getRank()), b);
  }

  // A GEMM operand as a rank-3 ABI buffer: leading dims collapsed into one
  // batch dim (a rank-2 operand is a batch of one), then, if transposed, the
  // view with the last two dims swapped.
  Value gemmOperand(Location loc, const GemmOperand &o) {
    auto tt = cast<RankedTensorType>(o.tensor.getType());
    auto s = tt.getShape();
    const int64_t r = tt.getRank();
    int64_t batch = 1;
    for (int64_t i = 0; i + 2 < r; ++i) batch *= s[i];
    Value b = reshaped(loc, dense(loc, o.tensor), {batch, s[r - 2], s[r - 1]});
    if (o.transposed) {
      auto map = AffineMap::getPermutationMap(ArrayRef<unsigned>{0, 2, 1}, rewriter.getContext());
      b = rewriter.create<memref::TransposeOp>(loc, b, AffineMapAttr::get(map));
    }
    return toAbi(loc, b);
  }

  // A fresh result buffer of tensor type `t`.
  Value alloc(Location loc, RankedTensorType t) {
    return rewriter.create<memref::AllocOp>(loc, MemRefType::get(t.getShape(), t.getElementType()));
  }

  Value asTensor(Location loc, Value buffer, Type tensorType) {
    return rewriter.create<bufferization::ToTensorOp>(loc, tensorType, buffer,
                                                      /*restrict=*/true, /*writable=*/true);
  }

  Value i32Const(Location loc, int64_t v) {
    return rewriter.create<arith::ConstantOp>(loc, rewriter.getI32IntegerAttr((int32_t)v));
  }

  // ---- callees -------------------------------------------------------------

  FunctionType sig(ArrayRef<Type> args) {
    return rewriter.getFunctionType(args, {rewriter.getI32Type()});
  }

  // Whether @name can be called with `type`: not yet declared, or declared
  // with that type (one module declares each entry point once).
  bool declarable(StringRef name, FunctionType type) {
    if (auto f = module.lookupSymbol<func::FuncOp>(name)) return f.getFunctionType() == type;
    return !module.lookupSymbol(name);
  }

  func::FuncOp declare(StringRef name, FunctionType type) {
    if (auto f = module.lookupSymbol<func::FuncOp>(name)) return f;
    OpBuilder::InsertionGuard guard(rewriter);
    rewriter.setInsertionPointToStart(module.getBody());
    auto f = rewriter.create<func::FuncOp>(module.getLoc(), name, type);
    f.setPrivate();
    f->setAttr(LLVM::LLVMDialect::getEmitCWrapperAttrName(), rewriter.getUnitAttr());
    return f;
  }

  // func.call @name(args) -> i32, then an assertion that it returned 0.
  void call(Location loc, StringRef name, ValueRange args) {
    SmallVector<Type> types;
    for (Value a : args) types.push_back(a.getType());
    auto c = rewriter.create<func::CallOp>(loc, declare(name, sig(types)), args);
    Value ok = rewriter.create<arith::CmpIOp>(loc, arith::CmpIPredicate::eq, c.getResult(0),
                                              i32Const(loc, NOVA_HIP_SUCCESS));
    rewriter.create<cf::AssertOp>(loc, ok, ("libnova_hip " + name + " failed").str());
  }

  Type f32() { return rewriter.getF32Type(); }
  Type i32() { return rewriter.getI32Type(); }

  // Index / label widening: the callee it needs (empty for i32) and its type.
  std::string widenName(int dt) {
    return dt == NOVA_HIP_DT_I16 ? "nova_hip_index_to_i32_i16"
           : dt == NOVA_HIP_DT_I64 ? "nova_hip_index_to_i32_i64" : "";
  }
  bool widenDeclarable(Value idx) {
    Type el = getElementTypeOrSelf(idx.getType());
    const std::string n = widenName(dtypeCode(el));
    return n.empty() || declarable(n, sig({abiType(el, 1), abiType(i32(), 1), i32()}));
  }
  // Indices as a flat i32 ABI buffer (non-i32 types widened on the GPU).
  Value indicesI32(Location loc, Value idx) {
    auto tt = cast<RankedTensorType>(idx.getType());
    const int64_t n = tt.getNumElements();
    Value flat = toAbi(loc, reshaped(loc, dense(loc, idx), {n}));
    const int dt = dtypeCode(tt.getElementType());
    if (dt == NOVA_HIP_DT_I32) return flat;
    Value wide = toAbi(loc, alloc(loc, RankedTensorType::get({n}, i32())));
    call(loc, widenName(dt), {flat, wide, i32Const(loc, dt)});
    return wide;
  }

  // Row-major [R, D] view of a tensor's dense buffer (leading dims folded).
  Value rows2d(Location loc, Value t) {
    auto tt = cast<RankedTensorType>(t.getType());
    const int64_t D = tt.getShape().back();
    return toAbi(loc, reshaped(loc, dense(loc, t), {tt.getNumElements() / D, D}));
  }
  Value flat1d(Location loc, Value t) {
    auto tt = cast<RankedTensorType>(t.getType());
    return toAbi(loc, reshaped(loc, dense(loc, t), {tt.getNumElements()}));
  }

  // Replace `result` by the buffer `buf` of the same element count, viewed
  // with the result's shape.
  void replaceWith(Location loc, Value result, Value buf) {
    auto rt = cast<RankedTensorType>(result.getType());
    auto bt = cast<MemRefType>(buf.getType());
    Value b = buf;
    if (bt.getShape() != rt.getShape()) {
      // dense [..] -> dense [rt shape]: a fresh identity-layout view
      SmallVector<ReassociationIndices> all(1);
      for (int64_t i = 0; i < bt.getRank(); ++i) all[0].push_back(i);
      Value flat = bt.getRank() == 1 ? buf : rewriter.create<memref::CollapseShapeOp>(loc, buf, all);
      SmallVector<ReassociationIndices> back(1);
      for (int64_t i = 0; i < rt.getRank(); ++i) back[0].push_back(i);
      if (rt.getRank() == 0) {
        b = rewriter.create<memref::CollapseShapeOp>(loc, flat, SmallVector<ReassociationIndices>{});
      } else {
        b = rewriter.create<memref::ExpandShapeOp>(
            loc, MemRefType::get(rt.getShape(), rt.getElementType()), flat, back);
      }
    }
    rewriter.replaceAllUsesWith(result, asTensor(loc, b, rt));
  }

  // ---- GEMMs -----------------------------------------------------------------

  // Entry-point name suffix of a dtype combination.  A module declares each
  // function once, with one type, but the generic entry points take operands
  // of any dtype; nova_hip.h therefore exports one alias per (input,
  // output[, bias]) dtype combination, which these names select.
  static std::string typeSuffix(int in, int out, int bias) {
    static const char *n[] = {"f32", "bf16", "f16"};
    std::string s = std::string(n[in]) + "_" + n[out];
    if (bias >= 0) s += std::string("_b") + n[bias];
    return s;
  }

  // nova.linear / nova.matmul / linalg.(batch_)matmul and their epilogue folds.
  LogicalResult lowerGemm(Operation *op, const char *form_name, Value lhs, Value rhs, Value bias,
                          Value outs) {
    Location loc = op->getLoc();
    Value result = op->getResult(0);
    auto rt = staticTensor(result);
    GemmOperand a = traceOperand(lhs), b = traceOperand(rhs);
    GemmOperand bo;
    if (bias) bo = traceOperand(bias);
    Form f;
    f.add(lhs, a.stored);
    f.add(rhs, b.stored);
    if (bias) f.add(bias, bo.stored);
    if (outs) f.add(outs);
    // linalg outs: a zero fill (the product overwrites it) or data the sums
    // start from (NOVA_HIP_GEMM_ACC_C); an uninitialised tensor.empty is
    // neither.
    bool accInto = false;
    if (outs) {
      bool zeroFill = false;
      if (auto fill = outs.getDefiningOp<linalg::FillOp>()) {
        auto c = fill.getInputs()[0].getDefiningOp<arith::ConstantOp>();
        auto fa = c ? dyn_cast<FloatAttr>(c.getValue()) : FloatAttr();
        zeroFill = fa && fa.getValue().isZero();
        if (!zeroFill) return failure();  // a non-zero fill: not on this path
      }
      if (!zeroFill && outs.getDefiningOp<tensor::EmptyOp>()) return failure();
      accInto = !zeroFill;
    }
    nova_forms::Attrs at;
    at.outs_zero = !accInto;
    if (!rt || declined(op, form_name, f, at)) return failure();
    if (bias && bo.transposed) return failure();  // a 1-D bias has no transpose
    if (outs) {
      if (auto mm = dyn_cast<linalg::MatmulOp>(op))
        if (mm.getIndexingMapsArray() != linalg::MatmulOp::getDefaultIndexingMaps(op->getContext()))
          return failure();
      if (auto bm = dyn_cast<linalg::BatchMatmulOp>(op))
        if (bm.getIndexingMapsArray() !=
            linalg::BatchMatmulOp::getDefaultIndexingMaps(op->getContext()))
          return failure();
    }
    const int in = dtypeCode(a.stored);
    int out = dtypeCode(rt.getElementType());
    const bool narrow = out != NOVA_HIP_DT_F32;
    int epi = bias ? NOVA_HIP_EPI_BIAS : NOVA_HIP_EPI_NONE;
    Operation *last = op;
    SmallVector<Operation *> folded;
    if (!narrow && !accInto) {
      if (Value u = singleUse(result)) {
        Operation *user = *u.getUsers().begin();
        if (auto g = dyn_cast<GeluOp>(user)) {
          epi = bias ? NOVA_HIP_EPI_BIAS_GELU : NOVA_HIP_EPI_GELU;
          folded.push_back(g);
          last = g;
        }
      }
      if (Value u = singleUse(last->getResult(0))) {
        if (auto c = dyn_cast<CastOp>(*u.getUsers().begin())) {
          const int to = dtypeCode(getElementTypeOrSelf(c.getType()));
          if (to == NOVA_HIP_DT_BF16 || to == NOVA_HIP_DT_F16) {
            out = to;
            folded.push_back(c);
            last = c;
          }
        }
      }
    }
    const int biasDt = bias ? dtypeCode(bo.stored) : NOVA_HIP_DT_F32;
    auto outTy = cast<RankedTensorType>(last->getResult(0).getType());
    const std::string name = "nova_hip_gemm_" + typeSuffix(in, out, biasDt);
    FunctionType ft = sig({abiType(a.stored, 3), abiType(b.stored, 3),
                           abiType(outTy.getElementType(), 3),
                           abiType(bias ? bo.stored : f32(), 1), i32()});
    if (!declarable(name, ft)) return failure();

    // Every check has passed: build.
    rewriter.setInsertionPoint(last);
    Value A = gemmOperand(loc, a), B = gemmOperand(loc, b);
    Value cBuf = alloc(loc, outTy);
    // Summing into a copy of outs' data keeps the outs tensor's own value.
    if (accInto) rewriter.create<memref::CopyOp>(loc, dense(loc, outs), cBuf);
    auto cs = outTy.getShape();
    const int64_t r = outTy.getRank();
    int64_t batch = 1;
    for (int64_t i = 0; i + 2 < r; ++i) batch *= cs[i];
    Value C = toAbi(loc, reshaped(loc, cBuf, {batch, cs[r - 2], cs[r - 1]}));
    // The entry point takes a bias descriptor always; an empty one when the
    // epilogue has none.
    Value biasAbi = bias ? flat1d(loc, bo.tensor)
                         : toAbi(loc, alloc(loc, RankedTensorType::get({0}, f32())));
    int32_t flags = NOVA_HIP_GEMM_FLAGS(in, out, epi, bias ? biasDt : 0);
    if (narrow) flags |= NOVA_HIP_GEMM_ACC_OUT;
    if (accInto) flags |= NOVA_HIP_GEMM_ACC_C;  // the exact kernel, from cBuf's data
    else if (in == NOVA_HIP_DT_F32 && f32Mfma) flags |= NOVA_HIP_GEMM_F32_MFMA;
    call(loc, name, {A, B, C, biasAbi, i32Const(loc, flags)});
    rewriter.replaceAllUsesWith(last->getResult(0), asTensor(loc, cBuf, outTy));
    for (auto it = folded.rbegin(); it != folded.rend(); ++it) {
      erasedOps.insert(*it);
      rewriter.eraseOp(*it);
    }
    rewriter.eraseOp(op);
    return success();
  }

  // nova.linear_backward / nova.matmul_backward: GEMMs over views, leading
  // dims of grad_out and input folded into rows.
  template <typename OpTy>
  LogicalResult lowerGemmBackward(OpTy op, const char *form_name, Value go, Value x, Value w,
                                  bool linear) {
    Location loc = op.getLoc();
    GemmOperand g = traceOperand(go), xi = traceOperand(x), wi = traceOperand(w);
    Form f;
    f.add(go, g.stored);
    f.add(x, xi.stored);
    f.add(w, wi.stored);
    if (declined(op, form_name, f)) return failure();
    if (g.transposed || xi.transposed || wi.transposed) return failure();
    const int in = dtypeCode(xi.stored);
    const int out = NOVA_HIP_DT_F32;  // the table admits f32 results only
    const std::string name =
        std::string(linear ? "nova_hip_linear_backward_" : "nova_hip_matmul_backward_") +
        typeSuffix(in, out, -1);
    SmallVector<Type> argTypes = {abiType(xi.stored, 2), abiType(xi.stored, 2),
                                  abiType(xi.stored, 2), abiType(f32(), 2), abiType(f32(), 2)};
    if (linear) argTypes.push_back(abiType(f32(), 1));
    argTypes.push_back(i32());
    if (!declarable(name, sig(argTypes))) return failure();

    rewriter.setInsertionPoint(op);
    SmallVector<Value> bufs, outs;
    for (Value r : op->getResults()) {
      Value buf = alloc(loc, cast<RankedTensorType>(r.getType()));
      bufs.push_back(buf);
      outs.push_back(toAbi(loc, buf));
    }
    // grad_input [..., M, K] is written as [rows, K]: its buffer viewed 2-D.
    {
      auto t = cast<RankedTensorType>(op->getResult(0).getType());
      const int64_t K = t.getShape().back();
      outs[0] = toAbi(loc, reshaped(loc, bufs[0], {t.getNumElements() / K, K}));
    }
    int32_t flags = NOVA_HIP_GEMM_FLAGS(in, out, NOVA_HIP_EPI_NONE, 0);
    if (in == NOVA_HIP_DT_F32 && f32Mfma) flags |= NOVA_HIP_GEMM_F32_MFMA;
    SmallVector<Value> args = {rows2d(loc, g.tensor), rows2d(loc, xi.tensor),
                               toAbi(loc, dense(loc, wi.tensor))};
    args.append(outs.begin(), outs.end());
    args.push_back(i32Const(loc, flags));
    call(loc, name, args);
    for (auto [r, b] : llvm::zip(op->getResults(), bufs))
      rewriter.replaceAllUsesWith(r, asTensor(loc, b, r.getType()));
    rewriter.eraseOp(op);
    return success();
  }

  // ---- row reductions ---------------------------------------------------------

  // nova.layer_norm -> (y, mean_sum, rstd); eps is the op's 1e-5
  // (NovaToLinalgGeneric.cpp:2025).
  LogicalResult lowerLayerNorm(LayerNormOp op) {
    Location loc = op.getLoc();
    Form f;
    f.add(op.getInput());
    f.add(op.getGamma());
    f.add(op.getBeta());
    if (declined(op, "nova.layer_norm", f)) return failure();
    const std::string name = "nova_hip_layer_norm_f32";
    if (!declarable(name, sig({abiType(f32(), 2), abiType(f32(), 1), abiType(f32(), 1),
                               abiType(f32(), 2), abiType(f32(), 1), abiType(f32(), 1), f32()})))
      return failure();
    auto xt = cast<RankedTensorType>(op.getInput().getType());
    const int64_t D = xt.getShape().back(), R = xt.getNumElements() / D;
    rewriter.setInsertionPoint(op);
    Value yBuf = alloc(loc, RankedTensorType::get({R, D}, f32()));
    Value sBuf = alloc(loc, RankedTensorType::get({R}, f32()));
    Value rBuf = alloc(loc, RankedTensorType::get({R}, f32()));
    Value eps = rewriter.create<arith::ConstantOp>(loc, rewriter.getF32FloatAttr(1.0e-5f));
    call(loc, name,
         {rows2d(loc, op.getInput()), flat1d(loc, op.getGamma()), flat1d(loc, op.getBeta()),
          toAbi(loc, yBuf), toAbi(loc, sBuf), toAbi(loc, rBuf), eps});
    replaceWith(loc, op.getOutput(), yBuf);
    replaceWith(loc, op.getMeanSum(), sBuf);
    replaceWith(loc, op.getVarSum(), rBuf);
    rewriter.eraseOp(op);
    return success();
  }

  // nova.sce (+ the nova.sce_backward of its softmax, fused).
  LogicalResult lowerSce(SceOp op) {
    Location loc = op.getLoc();
    Form f;
    f.add(op.getLogits());
    f.add(op.getTargets());
    if (declined(op, "nova.sce", f)) return failure();
    auto lt = cast<RankedTensorType>(op.getLogits().getType());
    SceBackwardOp bw;
    if (Value u = singleUse(op.getSoftmax()))
      if (auto b = dyn_cast<SceBackwardOp>(*u.getUsers().begin()))
        if (b.getTargets() == op.getTargets() &&
            (b.getDim() == -1 || b.getDim() == lt.getRank() - 1))
          bw = b;
    const bool smDead = op.getSoftmax().use_empty();
    const std::string name = bw ? "nova_hip_sce_fwd_bwd_f32"
                             : smDead ? "nova_hip_sce_loss_f32" : "nova_hip_sce_f32";
    SmallVector<Type> argTypes = {abiType(f32(), 2), abiType(i32(), 1), abiType(f32(), 1)};
    if (!smDead || bw) argTypes.push_back(abiType(f32(), 2));
    if (!declarable(name, sig(argTypes)) || !widenDeclarable(op.getTargets())) return failure();

    const int64_t C = lt.getShape().back(), R = lt.getNumElements() / C;
    rewriter.setInsertionPoint(bw ? bw.getOperation() : op.getOperation());
    Value x = rows2d(loc, op.getLogits());
    Value t = indicesI32(loc, op.getTargets());
    Value lossBuf = alloc(loc, RankedTensorType::get({1}, f32()));
    auto full = RankedTensorType::get({R, C}, f32());
    if (bw) {
      Value gBuf = alloc(loc, full);
      call(loc, name, {x, t, toAbi(loc, lossBuf), toAbi(loc, gBuf)});
      replaceWith(loc, bw.getGradLogits(), gBuf);
      erasedOps.insert(bw);
      rewriter.eraseOp(bw);
    } else if (smDead) {
      // The op is Pure and its softmax dead: the loss alone.
      call(loc, name, {x, t, toAbi(loc, lossBuf)});
    } else {
      Value smBuf = alloc(loc, full);
      call(loc, name, {x, t, toAbi(loc, lossBuf), toAbi(loc, smBuf)});
      replaceWith(loc, op.getSoftmax(), smBuf);
    }
    replaceWith(loc, op.getResult(), lossBuf);
    rewriter.eraseOp(op);
    return success();
  }

  // nova.sce_backward on its own.
  LogicalResult lowerSceBackward(SceBackwardOp op) {
    Location loc = op.getLoc();
    Form f;
    f.add(op.getSoftmax());
    f.add(op.getTargets());
    nova_forms::Attrs at;
    if (auto st = staticTensor(op.getSoftmax())) {
      int64_t d = op.getDim();
      if (d < 0) d += st.getRank();
      at.dim = d == st.getRank() - 1 ? -1 : (int)d;
    }
    if (declined(op, "nova.sce_backward", f, at)) return failure();
    const std::string name = "nova_hip_sce_backward_f32";
    if (!declarable(name, sig({abiType(f32(), 2), abiType(i32(), 1), abiType(f32(), 2)})) ||
        !widenDeclarable(op.getTargets()))
      return failure();
    auto st = cast<RankedTensorType>(op.getSoftmax().getType());
    const int64_t C = st.getShape().back(), R = st.getNumElements() / C;
    rewriter.setInsertionPoint(op);
    Value t = indicesI32(loc, op.getTargets());
    Value gBuf = alloc(loc, RankedTensorType::get({R, C}, f32()));
    call(loc, name, {rows2d(loc, op.getSoftmax()), t, toAbi(loc, gBuf)});
    replaceWith(loc, op.getGradLogits(), gBuf);
    rewriter.eraseOp(op);
    return success();
  }

  // nova.layer_norm_backward with the forward's saved stats.
  LogicalResult lowerLayerNormBackward(LayerNormBackwardOp op) {
    Location loc = op.getLoc();
    Form f;
    for (Value v : {op.getGradY(), op.getX(), op.getGamma(), op.getMeanSum(), op.getVarSum()})
      f.add(v);
    if (declined(op, "nova.layer_norm_backward", f)) return failure();
    const std::string name = "nova_hip_layer_norm_backward_f32";
    if (!declarable(name, sig({abiType(f32(), 2), abiType(f32(), 2), abiType(f32(), 1),
                               abiType(f32(), 1), abiType(f32(), 1), abiType(f32(), 2),
                               abiType(f32(), 1), abiType(f32(), 1)})))
      return failure();
    auto xt = cast<RankedTensorType>(op.getX().getType());
    const int64_t D = xt.getShape().back(), R = xt.getNumElements() / D;
    rewriter.setInsertionPoint(op);
    Value dxBuf = alloc(loc, RankedTensorType::get({R, D}, f32()));
    Value dgBuf = alloc(loc, RankedTensorType::get({D}, f32()));
    Value dbBuf = alloc(loc, RankedTensorType::get({D}, f32()));
    call(loc, name,
         {rows2d(loc, op.getGradY()), rows2d(loc, op.getX()), flat1d(loc, op.getGamma()),
          flat1d(loc, op.getMeanSum()), flat1d(loc, op.getVarSum()), toAbi(loc, dxBuf),
          toAbi(loc, dgBuf), toAbi(loc, dbBuf)});
    replaceWith(loc, op.getGradX(), dxBuf);
    replaceWith(loc, op.getGradGamma(), dgBuf);
    replaceWith(loc, op.getGradBeta(), dbBuf);
    rewriter.eraseOp(op);
    return success();
  }

  // ---- program glue -------------------------------------------------------------

  // nova.add / sub / mul / div: operands and result as 4-D views (leading
  // unit dims), size-1 dims broadcast by the entry point.
  LogicalResult lowerBinary(Operation *op, const char *form_name, int code) {
    Location loc = op->getLoc();
    Value a = op->getOperand(0), b = op->getOperand(1), r = op->getResult(0);
    Form f;
    f.add(a);
    f.add(b);
    auto rt = staticTensor(r);
    if (!rt || declined(op, form_name, f)) return failure();
    const std::string name = "nova_hip_binary_f32";
    if (!declarable(name, sig({abiType(f32(), 4), abiType(f32(), 4), abiType(f32(), 4), i32()})))
      return failure();
    auto four = [&](Value buf, ArrayRef<int64_t> s) {
      SmallVector<int64_t> s4(4 - s.size(), 1);
      s4.append(s.begin(), s.end());
      return toAbi(loc, reshaped(loc, buf, s4));
    };
    rewriter.setInsertionPoint(op);
    Value cBuf = alloc(loc, rt);
    call(loc, name,
         {four(dense(loc, a), cast<RankedTensorType>(a.getType()).getShape()),
          four(dense(loc, b), cast<RankedTensorType>(b.getType()).getShape()),
          four(cBuf, rt.getShape()), i32Const(loc, code)});
    rewriter.replaceAllUsesWith(r, asTensor(loc, cBuf, rt));
    rewriter.eraseOp(op);
    return success();
  }

  // nova.gelu that did not fold into a GEMM epilogue, and nova.gelu_backward:
  // flat [n] streams.
  LogicalResult lowerGelu(Operation *op, bool backward) {
    Location loc = op->getLoc();
    Form f;
    for (Value v : op->getOperands()) f.add(v);
    auto rt = staticTensor(op->getResult(0));
    if (!rt || declined(op, backward ? "nova.gelu_backward" : "nova.gelu", f)) return failure();
    const std::string name = backward ? "nova_hip_gelu_backward_f32" : "nova_hip_gelu_f32";
    SmallVector<Type> argTypes(backward ? 3 : 2, abiType(f32(), 1));
    if (!declarable(name, sig(argTypes))) return failure();
    rewriter.setInsertionPoint(op);
    Value outBuf = alloc(loc, rt);
    SmallVector<Value> args;
    for (Value v : op->getOperands()) args.push_back(flat1d(loc, v));
    args.push_back(toAbi(loc, reshaped(loc, outBuf, {rt.getNumElements()})));
    call(loc, name, args);
    rewriter.replaceAllUsesWith(op->getResult(0), asTensor(loc, outBuf, rt));
    rewriter.eraseOp(op);
    return success();
  }

  // A splat f32 nova.constant: a fill.
  LogicalResult lowerConstant(ConstantOp op) {
    Location loc = op.getLoc();
    auto rt = staticTensor(op.getResult());
    auto attr = dyn_cast<DenseElementsAttr>(op.getValue());
    nova_forms::Attrs at;
    at.splat_f32 = rt && attr && attr.isSplat() && rt.getElementType().isF32();
    Form f;
    if (declined(op, "nova.constant", f, at)) return failure();
    const std::string name = "nova_hip_fill_f32";
    if (!declarable(name, sig({abiType(f32(), 1), f32()}))) return failure();
    rewriter.setInsertionPoint(op);
    Value buf = alloc(loc, rt);
    Value v = rewriter.create<arith::ConstantOp>(loc, attr.getSplatValue<FloatAttr>());
    call(loc, name, {toAbi(loc, reshaped(loc, buf, {rt.getNumElements()})), v});
    rewriter.replaceAllUsesWith(op.getResult(), asTensor(loc, buf, rt));
    rewriter.eraseOp(op);
    return success();
  }

  // nova.gather along axis 0 (the embedding lookup): table [V, D], indices
  // flattened and widened to i32, out [n, D] viewed as the result shape.
  LogicalResult lowerGather(GatherOp op) {
    Location loc = op.getLoc();
    Form f;
    f.add(op.getInput());
    f.add(op.getIndices());
    nova_forms::Attrs at;
    at.axis = (int)op.getAxis();
    if (auto t = staticTensor(op.getInput()))
      if (at.axis < 0) at.axis += (int)t.getRank();
    auto rt = staticTensor(op.getResult());
    if (!rt || declined(op, "nova.gather", f, at)) return failure();
    const std::string name = "nova_hip_gather_f32";
    if (!declarable(name, sig({abiType(f32(), 2), abiType(i32(), 1), abiType(f32(), 2), i32()})) ||
        !widenDeclarable(op.getIndices()))
      return failure();
    rewriter.setInsertionPoint(op);
    auto tt = cast<RankedTensorType>(op.getInput().getType());
    const int64_t D = tt.getShape()[1];
    Value idx = indicesI32(loc, op.getIndices());
    Value outBuf = alloc(loc, rt);
    call(loc, name,
         {toAbi(loc, dense(loc, op.getInput())), idx,
          toAbi(loc, reshaped(loc, outBuf, {rt.getNumElements() / D, D})),
          i32Const(loc, NOVA_HIP_DT_I32)});
    rewriter.replaceAllUsesWith(op.getResult(), asTensor(loc, outBuf, rt));
    rewriter.eraseOp(op);
    return success();
  }

  // nova.scatter_add along axis 0: the input copied into a fresh buffer, then
  // the adds into it.
  LogicalResult lowerScatterAdd(ScatterAddOp op) {
    Location loc = op.getLoc();
    Form f;
    f.add(op.getInput());
    f.add(op.getIndices());
    f.add(op.getSrc());
    nova_forms::Attrs at;
    at.axis = (int)op.getAxis();
    if (auto t = staticTensor(op.getInput()))
      if (at.axis < 0) at.axis += (int)t.getRank();
    auto rt = staticTensor(op.getResult());
    if (!rt || declined(op, "nova.scatter_add", f, at)) return failure();
    const std::string name = "nova_hip_scatter_add_f32";
    if (!declarable(name, sig({abiType(f32(), 2), abiType(i32(), 1), abiType(f32(), 2), i32()})) ||
        !widenDeclarable(op.getIndices()))
      return failure();
    rewriter.setInsertionPoint(op);
    const int64_t D = rt.getShape()[1];
    Value outBuf = alloc(loc, rt);
    rewriter.create<memref::CopyOp>(loc, dense(loc, op.getInput()), outBuf);
    Value idx = indicesI32(loc, op.getIndices());
    auto srcT = cast<RankedTensorType>(op.getSrc().getType());
    call(loc, name,
         {toAbi(loc, outBuf), idx,
          toAbi(loc, reshaped(loc, dense(loc, op.getSrc()), {srcT.getNumElements() / D, D})),
          i32Const(loc, NOVA_HIP_DT_I32)});
    rewriter.replaceAllUsesWith(op.getResult(), asTensor(loc, outBuf, rt));
    rewriter.eraseOp(op);
    return success();
  }

  // nova.reduce<sum> over adjacent dims: x viewed as [outer, n, inner].
  LogicalResult lowerReduceSum(ReduceOp op) {
    Location loc = op.getLoc();
    auto xt = staticTensor(op.getInput());
    auto rt = staticTensor(op.getResult());
    Form f;
    f.add(op.getInput());
    nova_forms::Attrs at;
    at.ignore_nan = op.getIgnoreNan();
    SmallVector<int64_t> dims;
    if (xt) {
      if (auto d = op.getDimension())
        for (Attribute a : *d) {
          int64_t v = cast<IntegerAttr>(a).getInt();
          dims.push_back(v < 0 ? v + xt.getRank() : v);
        }
      else
        for (int64_t i = 0; i < xt.getRank(); ++i) dims.push_back(i);
      llvm::sort(dims);
      for (size_t i = 1; i < dims.size(); ++i) at.adjacent = at.adjacent && dims[i] == dims[i - 1] + 1;
    }
    const bool sum = op.getKind() == ReductionKind::SUM;
    if (!rt || !sum || dims.empty() || declined(op, "nova.reduce<sum>", f, at)) return failure();
    const std::string name = "nova_hip_reduce_sum_f32";
    if (!declarable(name, sig({abiType(f32(), 3), abiType(f32(), 2)}))) return failure();
    auto s = xt.getShape();
    int64_t outer = 1, n = 1, inner = 1;
    for (int64_t i = 0; i < xt.getRank(); ++i)
      (i < dims.front() ? outer : i <= dims.back() ? n : inner) *= s[i];
    rewriter.setInsertionPoint(op);
    Value outBuf = alloc(loc, rt);
    call(loc, name,
         {toAbi(loc, reshaped(loc, dense(loc, op.getInput()), {outer, n, inner})),
          toAbi(loc, reshaped(loc, outBuf, {outer, inner}))});
    rewriter.replaceAllUsesWith(op.getResult(), asTensor(loc, outBuf, rt));
    rewriter.eraseOp(op);
    return success();
  }

  void run() {
    SmallVector<Operation *> work;
    module.walk([&](Operation *op) {
      if (isa<LinearOp, MatmulOp, LayerNormOp, SceOp, SceBackwardOp, LayerNormBackwardOp,
              LinearBackwardOp, MatmulBackwardOp, linalg::MatmulOp, linalg::BatchMatmulOp,
              AddOp, SubOp, MulOp, DivOp, GeluOp, GeluBackwardOp, ConstantOp, GatherOp,
              ScatterAddOp, ReduceOp>(op))
        work.push_back(op);
    });
    for (Operation *op : work) {
      // (a sce_backward fused into its nova.sce is gone, and so is a gelu
      // folded into its GEMM's epilogue)
      if (erasedOps.contains(op)) continue;
      (void)llvm::TypeSwitch<Operation *, LogicalResult>(op)
          .Case([&](LinearOp o) {
            return lowerGemm(o, "nova.linear", o.getInput(), o.getWeight(), o.getBias(), Value());
          })
          .Case([&](MatmulOp o) {
            return lowerGemm(o, "nova.matmul", o.getLhs(), o.getRhs(), Value(), Value());
          })
          .Case([&](linalg::MatmulOp o) {
            return lowerGemm(o, "linalg.matmul", o.getDpsInputs()[0], o.getDpsInputs()[1], Value(),
                             o.getDpsInits()[0]);
          })
          .Case([&](linalg::BatchMatmulOp o) {
            return lowerGemm(o, "linalg.batch_matmul", o.getDpsInputs()[0], o.getDpsInputs()[1],
                             Value(), o.getDpsInits()[0]);
          })
          .Case([&](LayerNormOp o) { return lowerLayerNorm(o); })
          .Case([&](SceOp o) { return lowerSce(o); })
          .Case([&](SceBackwardOp o) { return lowerSceBackward(o); })
          .Case([&](LayerNormBackwardOp o) { return lowerLayerNormBackward(o); })
          .Case([&](LinearBackwardOp o) {
            return lowerGemmBackward(o, "nova.linear_backward", o.getGradOut(), o.getInput(),
                                     o.getWeight(), true);
          })
          .Case([&](MatmulBackwardOp o) {
            return lowerGemmBackward(o, "nova.matmul_backward", o.getGradOut(), o.getA(), o.getB(),
                                     false);
          })
          .Case([&](AddOp o) { return lowerBinary(o, "nova.add", NOVA_HIP_BIN_ADD); })
          .Case([&](SubOp o) { return lowerBinary(o, "nova.sub", NOVA_HIP_BIN_SUB); })
          .Case([&](MulOp o) { return lowerBinary(o, "nova.mul", NOVA_HIP_BIN_MUL); })
          .Case([&](DivOp o) { return lowerBinary(o, "nova.div", NOVA_HIP_BIN_DIV); })
          .Case([&](GeluOp o) { return lowerGelu(o, false); })
          .Case([&](GeluBackwardOp o) { return lowerGelu(o, true); })
          .Case([&](ConstantOp o) { return lowerConstant(o); })
          .Case([&](GatherOp o) { return lowerGather(o); })
          .Case([&](ScatterAddOp o) { return lowerScatterAdd(o); })
          .Case([&](ReduceOp o) { return lowerReduceSum(o); })
          .Default([](Operation *) { return failure(); });
    }
  }

  // Nova ops still in the module that would become kernels on the existing
  // (NVPTX) path: every remaining op of the dialect with uses, except
  // nova.reshape (a tensor view).
  SmallVector<Operation *> leftovers() {
    SmallVector<Operation *> left;
    module.walk([&](Operation *op) {
      if (op->getDialect() && op->getDialect()->getNamespace() == "nova" &&
          !isa<ReshapeOp>(op) && !op->use_empty())
        left.push_back(op);
    });
    return left;
  }

 private:
  ModuleOp module;
  IRRewriter rewriter;
  bool f32Mfma;
  llvm::SmallPtrSet<Operation *, 16> erasedOps;
};

struct NovaHipLoweringPass
    : public PassWrapper<NovaHipLoweringPass, OperationPass<ModuleOp>> {
  MLIR_DEFINE_EXPLICIT_INTERNAL_INLINE_TYPE_ID(NovaHipLoweringPass)

  NovaHipLoweringPass() = default;
  NovaHipLoweringPass(const NovaHipLoweringPass &other) : PassWrapper(other) {}

  StringRef getArgument() const final { return "nova-hip-lower"; }
  StringRef getDescription() const final {
    return "Rewrite Nova's matmul / linear / layer_norm / sce ops, their backward ops and "
           "the program glue into calls to libnova_hip's gfx950 kernels";
  }
  void getDependentDialects(DialectRegistry &registry) const override {
    registry.insert<arith::ArithDialect, bufferization::BufferizationDialect,
                    cf::ControlFlowDialect, func::FuncDialect, memref::MemRefDialect,
                    LLVM::LLVMDialect>();
  }

  Option<std::string> f32Gemm{*this, "f32-gemm",
                              llvm::cl::desc("f32 GEMMs: 'exact' (bit-identical to the CPU "
                                             "pipeline) or 'mfma' (f32 matrix cores, 1e-4)"),
                              llvm::cl::init("exact")};
  Option<bool> strict{*this, "strict",
                      llvm::cl::desc("fail on any Nova op left for the NVPTX path (which "
                                     "cannot run on AMD), with the form table's reason"),
                      llvm::cl::init(false)};

  void runOnOperation() override {
    if (f32Gemm != "exact" && f32Gemm != "mfma") {
      getOperation().emitError() << "nova-hip-lower: f32-gemm must be 'exact' or 'mfma'";
      return signalPassFailure();
    }
    Lowerer l(getOperation(), f32Gemm == "mfma");
    l.run();
    if (!strict) return;
    bool failed = false;
    llvm::SmallPtrSet<Operation *, 16> reported;
    for (auto &[op, why] : l.declinedOps) {
      if (!op->getBlock() || !reported.insert(op).second) continue;
      op->emitError() << "nova-hip-lower: not on the libnova_hip path: " << why;
      failed = true;
    }
    for (Operation *op : l.leftovers()) {
      if (reported.contains(op)) continue;
      op->emitError() << "nova-hip-lower: not on the libnova_hip path: "
                      << "not part of this path's op surface (or a view no lowered op folds)";
      failed = true;
    }
    if (failed) signalPassFailure();
  }
};

}  // namespace

std::unique_ptr<Pass> createNovaHipLoweringPass() {
  return std::make_unique<NovaHipLoweringPass>();
}

void registerNovaHipLoweringPass() { PassRegistration<NovaHipLoweringPass>(); }

}  // namespace mlir::nova
