//===- NovaHipLowering.cpp - Nova hot ops -> calls into libnova_hip -------===//
//
// The lowering that takes Nova's GPU matmul / reduction ops off the
// IREE-derived LLVMGPU sequence (lib/Transforms/LLVMGPU/Passes.cpp:115-372:
// TileAndDistribute, PromoteMatmulOperands, PadOperands, vector
// distribution, multibuffering) and calls the hand-written gfx950 kernels of
// libnova_hip instead.  It runs on the Nova ops themselves, ahead of
// Nova -> Linalg (Passes.cpp:88-90), so the ops it rewrites never reach that
// sequence; every other op, and every form below it declines, keeps the
// existing path.
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
// the C interface, whatever the static type.  One-shot bufferization later
// resolves the to_buffer / to_tensor pairs.
//
// The op forms and folds are those of the MLIR-free planner that carries the
// same rewrite in this repository (runtime/nova_run.cpp), one pattern each:
//   * nova.transpose of the last two dims feeding a GEMM operand is a
//     memref.transpose view (strided), not a copy;
//   * a widening nova.cast (bf16 / f16 -> f32) feeding a GEMM operand is
//     dropped: the kernel reads the narrow data and accumulates in f32;
//   * nova.linear / nova.matmul followed by a nova.gelu that is the result's
//     only use, and then a narrowing nova.cast that is the only use, fold
//     into the GEMM's epilogue (bias -> GELU -> round to bf16 / f16);
//   * bf16 / f16 GEMMs whose result keeps the narrow type accumulate in it
//     (NOVA_HIP_GEMM_ACC_OUT), as linalg.matmul with narrow outs does; a
//     bf16 x bf16 nova.matmul (f16 result, NovaOps.cpp:1198) is declined;
//   * nova.sce whose softmax feeds only a nova.sce_backward over the same
//     targets is one fused call, and the softmax is never materialised;
//   * non-i32 targets are widened by nova_hip_index_to_i32 first.
// f32 GEMMs run the exact kernel (bit-identical to the CPU pipeline) unless
// the pass option f32-gemm=mfma selects the f32 matrix cores.
//
// Built only where MLIR is available (CMakeLists.txt next to this file,
// find_package(MLIR)): this repository's image has none, so the planner is
// the tested carrier of the rewrite.
//===----------------------------------------------------------------------===//

#include "Compiler/Dialect/nova/NovaDialect.h"
#include "Compiler/Dialect/nova/NovaOps.h"

#include "mlir/Dialect/Arith/IR/Arith.h"
#include "mlir/Dialect/Bufferization/IR/Bufferization.h"
#include "mlir/Dialect/ControlFlow/IR/ControlFlowOps.h"
#include "mlir/Dialect/Func/IR/FuncOps.h"
#include "mlir/Dialect/LLVMIR/LLVMDialect.h"
#include "mlir/Dialect/MemRef/IR/MemRef.h"
#include "mlir/IR/AffineMap.h"
#include "mlir/IR/BuiltinOps.h"
#include "mlir/IR/PatternMatch.h"
#include "mlir/Pass/Pass.h"
#include "mlir/Pass/PassRegistry.h"
#include "llvm/ADT/SmallPtrSet.h"
#include "llvm/ADT/TypeSwitch.h"

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

bool staticRanked(Value v) {
  auto t = dyn_cast<RankedTensorType>(v.getType());
  return t && t.hasStaticShape();
}

Value singleUse(Value v) { return v.hasOneUse() ? v : Value(); }

// What a GEMM operand reads: the tensor holding the data (through a widening
// cast and a transpose of the last two dims), and whether it is transposed.
struct GemmOperand {
  Value tensor;
  bool transposed = false;
  Type stored;  // element type of the data read
};

GemmOperand traceOperand(Value v) {
  GemmOperand o;
  o.tensor = v;
  // f32 view of narrow data: nova.cast bf16 / f16 -> f32 (exact widening).
  if (auto c = v.getDefiningOp<CastOp>()) {
    Type from = getElementTypeOrSelf(c.getInput().getType());
    Type to = getElementTypeOrSelf(c.getType());
    if (to.isF32() && (from.isBF16() || from.isF16())) o.tensor = c.getInput();
  }
  // nova.transpose of the last two dims, before or after the cast.
  if (auto t = o.tensor.getDefiningOp<TransposeOp>()) {
    auto ty = cast<RankedTensorType>(t.getInput().getType());
    const int64_t r = ty.getRank();
    int64_t a1 = t.getAxes1(), a2 = t.getAxes2();
    if (a1 < 0) a1 += r;
    if (a2 < 0) a2 += r;
    if (r >= 2 && ((a1 == r - 1 && a2 == r - 2) || (a1 == r - 2 && a2 == r - 1))) {
      o.tensor = t.getInput();
      o.transposed = true;
      if (auto c = o.tensor.getDefiningOp<CastOp>()) {
        Type from = getElementTypeOrSelf(c.getInput().getType());
        if (getElementTypeOrSelf(c.getType()).isF32() && (from.isBF16() || from.isF16()))
          o.tensor = c.getInput();
      }
    }
  }
  o.stored = getElementTypeOrSelf(o.tensor.getType());
  return o;
}

class Lowerer {
 public:
  Lowerer(ModuleOp m, bool f32Mfma) : module(m), rewriter(m.getContext()), f32Mfma(f32Mfma) {}

  // Buffer of a tensor value, as the ABI memref type: optionally the
  // transposed view of its last two dims, and a rank-2 value optionally as
  // [1, M, N] (a batch of one, which the GEMM entry points broadcast).
  Value abiBuffer(Location loc, Value tensor, bool transposed = false, bool rank3 = false) {
    auto tt = cast<RankedTensorType>(tensor.getType());
    auto mt = MemRefType::get(tt.getShape(), tt.getElementType());
    Value b = rewriter.create<bufferization::ToBufferOp>(loc, mt, tensor, /*readOnly=*/true);
    const int64_t r = tt.getRank();
    if (transposed) {
      SmallVector<unsigned> perm;
      for (int64_t i = 0; i < r; ++i) perm.push_back((unsigned)i);
      std::swap(perm[r - 1], perm[r - 2]);
      auto map = AffineMap::getPermutationMap(perm, rewriter.getContext());
      b = rewriter.create<memref::TransposeOp>(loc, b, AffineMapAttr::get(map));
    }
    int64_t rank = r;
    if (rank3 && r == 2) b = batchOfOne(loc, b), rank = 3;
    return rewriter.create<memref::CastOp>(loc, abiType(tt.getElementType(), rank), b);
  }

  // [M, N] (any strided layout) -> [1, M, N].
  Value batchOfOne(Location loc, Value b) {
    auto mt = cast<MemRefType>(b.getType());
    SmallVector<ReassociationIndices> re = {{0, 1}, {2}};
    SmallVector<int64_t> shape = {1, mt.getShape()[0], mt.getShape()[1]};
    FailureOr<MemRefType> et = memref::ExpandShapeOp::computeExpandedType(mt, shape, re);
    return rewriter.create<memref::ExpandShapeOp>(loc, *et, b, re);
  }

  // A fresh result buffer of tensor type `t`; `abi` receives its ABI view.
  Value allocResult(Location loc, RankedTensorType t, Value &abi) {
    Value m = rewriter.create<memref::AllocOp>(
        loc, MemRefType::get(t.getShape(), t.getElementType()));
    abi = rewriter.create<memref::CastOp>(loc, abiType(t.getElementType(), t.getRank()), m);
    return m;
  }

  Value asTensor(Location loc, Value buffer, Type tensorType) {
    return rewriter.create<bufferization::ToTensorOp>(loc, tensorType, buffer,
                                                      /*restrict=*/true, /*writable=*/true);
  }

  Value i32Const(Location loc, int64_t v) {
    return rewriter.create<arith::ConstantOp>(loc, rewriter.getI32IntegerAttr((int32_t)v));
  }

  // The private, C-interface declaration of @name, created on first use.
  // Null when the module already declares @name with another type (one
  // module calls each generic entry point with one operand type only).
  func::FuncOp declare(StringRef name, FunctionType type) {
    if (auto f = module.lookupSymbol<func::FuncOp>(name))
      return f.getFunctionType() == type ? f : func::FuncOp();
    OpBuilder::InsertionGuard guard(rewriter);
    rewriter.setInsertionPointToStart(module.getBody());
    auto f = rewriter.create<func::FuncOp>(module.getLoc(), name, type);
    f.setPrivate();
    f->setAttr(LLVM::LLVMDialect::getEmitCWrapperAttrName(), rewriter.getUnitAttr());
    return f;
  }

  // func.call @name(args) -> i32, then an assertion that it returned 0.
  LogicalResult call(Location loc, StringRef name, ValueRange args) {
    SmallVector<Type> types;
    for (Value a : args) types.push_back(a.getType());
    auto f = declare(name, rewriter.getFunctionType(types, {rewriter.getI32Type()}));
    if (!f) return failure();
    auto c = rewriter.create<func::CallOp>(loc, f, args);
    Value ok = rewriter.create<arith::CmpIOp>(loc, arith::CmpIPredicate::eq, c.getResult(0),
                                              i32Const(loc, NOVA_HIP_SUCCESS));
    rewriter.create<cf::AssertOp>(loc, ok, ("libnova_hip " + name + " failed").str());
    return success();
  }

  // Labels as an i32 buffer (non-i32 integer targets widened on the GPU).
  Value labelsI32(Location loc, Value targets) {
    auto tt = cast<RankedTensorType>(targets.getType());
    const int dt = dtypeCode(tt.getElementType());
    auto flat = [&](Value t) {
      auto ty = cast<RankedTensorType>(t.getType());
      Value b = abiBuffer(loc, t);
      if (ty.getRank() == 1) return b;
      // [d0, ..., dn] -> [d0 * ... * dn], a view of the dense buffer.
      SmallVector<ReassociationIndices> all(1);
      for (int64_t i = 0; i < ty.getRank(); ++i) all[0].push_back(i);
      Value dense = rewriter.create<bufferization::ToBufferOp>(
          loc, MemRefType::get(ty.getShape(), ty.getElementType()), t, true);
      Value c = rewriter.create<memref::CollapseShapeOp>(loc, dense, all);
      return rewriter.create<memref::CastOp>(loc, abiType(ty.getElementType(), 1), c)
          .getResult();
    };
    if (dt == NOVA_HIP_DT_I32) return flat(targets);
    if (dt != NOVA_HIP_DT_I16 && dt != NOVA_HIP_DT_I64) return Value();
    auto wide = RankedTensorType::get({tt.getNumElements()}, rewriter.getI32Type());
    Value abi;
    allocResult(loc, wide, abi);
    if (failed(call(loc, dt == NOVA_HIP_DT_I16 ? "nova_hip_index_to_i32_i16"
                                                : "nova_hip_index_to_i32_i64",
                    {flat(targets), abi, i32Const(loc, dt)})))
      return Value();
    return abi;
  }

  // nova.linear / nova.matmul (rank 2 or 3) and their epilogue folds.
  LogicalResult lowerGemm(Operation *op, Value lhs, Value rhs, Value bias) {
    Location loc = op->getLoc();
    Value result = op->getResult(0);
    auto rt = cast<RankedTensorType>(result.getType());
    if (!staticRanked(lhs) || !staticRanked(rhs) || !rt.hasStaticShape() || rt.getRank() > 3 ||
        rt.getRank() < 2)
      return failure();
    GemmOperand a = traceOperand(lhs), b = traceOperand(rhs);
    if (a.stored != b.stored) return failure();
    const int in = dtypeCode(a.stored);
    int out = dtypeCode(rt.getElementType());
    if (in < 0 || in > NOVA_HIP_DT_F16 || out < 0 || out > NOVA_HIP_DT_F16) return failure();
    // Narrow result: linalg.matmul with narrow outs accumulates in it; only
    // the same-dtype form is on this path.
    const bool narrow = out != NOVA_HIP_DT_F32;
    if (narrow && (in != out || getElementTypeOrSelf(lhs.getType()) != a.stored ||
                   getElementTypeOrSelf(rhs.getType()) != b.stored))
      return failure();
    int epi = bias ? NOVA_HIP_EPI_BIAS : NOVA_HIP_EPI_NONE;
    Operation *last = op;
    SmallVector<Operation *> folded;
    if (!narrow) {
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
    int biasDt = 0;
    GemmOperand bo;
    if (bias) {
      if (!staticRanked(bias)) return failure();
      bo = traceOperand(bias);
      biasDt = dtypeCode(bo.stored);
      if (biasDt < 0 || biasDt > NOVA_HIP_DT_F16 || (narrow && biasDt != in)) return failure();
    }
    rewriter.setInsertionPoint(last);
    auto outTy = cast<RankedTensorType>(last->getResult(0).getType());
    // Every GEMM goes through the 3-D entry point; a rank-2 operand or
    // result is a batch of one.
    Value A = abiBuffer(loc, a.tensor, a.transposed, /*rank3=*/true);
    Value B = abiBuffer(loc, b.tensor, b.transposed, /*rank3=*/true);
    Value cBuf = rewriter.create<memref::AllocOp>(
        loc, MemRefType::get(outTy.getShape(), outTy.getElementType()));
    Value C = cBuf;
    if (outTy.getRank() == 2) C = batchOfOne(loc, C);
    C = rewriter.create<memref::CastOp>(loc, abiType(outTy.getElementType(), 3), C);
    Value biasAbi;
    if (bias) {
      biasAbi = abiBuffer(loc, bo.tensor);
    } else {
      // The entry point takes a bias descriptor always; an empty one when
      // the epilogue has none.
      Value z;
      allocResult(loc, RankedTensorType::get({0}, rewriter.getF32Type()), z);
      biasAbi = z;
    }
    int32_t flags = NOVA_HIP_GEMM_FLAGS(in, out, epi, biasDt);
    if (narrow) flags |= NOVA_HIP_GEMM_ACC_OUT;
    if (in == NOVA_HIP_DT_F32 && f32Mfma) flags |= NOVA_HIP_GEMM_F32_MFMA;
    const std::string name = "nova_hip_gemm_" + typeSuffix(in, out, bias ? biasDt : NOVA_HIP_DT_F32);
    if (failed(call(loc, name, {A, B, C, biasAbi, i32Const(loc, flags)}))) return failure();
    rewriter.replaceAllUsesWith(last->getResult(0), asTensor(loc, cBuf, outTy));
    for (auto it = folded.rbegin(); it != folded.rend(); ++it) rewriter.eraseOp(*it);
    rewriter.eraseOp(op);
    return success();
  }

  // nova.layer_norm -> (y, mean_sum, rstd); eps is the op's 1e-5
  // (NovaToLinalgGeneric.cpp:2025).
  LogicalResult lowerLayerNorm(LayerNormOp op) {
    Location loc = op.getLoc();
    auto xt = dyn_cast<RankedTensorType>(op.getInput().getType());
    if (!xt || !xt.hasStaticShape() || xt.getRank() < 2 || !xt.getElementType().isF32())
      return failure();
    rewriter.setInsertionPoint(op);
    const int64_t D = xt.getShape().back(), R = xt.getNumElements() / D;
    // Rows flattened: [..., D] -> [R, D]; the stats [R].
    Value x = flat2d(loc, op.getInput(), R, D);
    Value yAbi, sAbi, rAbi;
    auto y2 = RankedTensorType::get({R, D}, rewriter.getF32Type());
    auto r1 = RankedTensorType::get({R}, rewriter.getF32Type());
    Value yBuf = allocResult(loc, y2, yAbi);
    Value sBuf = allocResult(loc, r1, sAbi);
    Value rBuf = allocResult(loc, r1, rAbi);
    Value eps = rewriter.create<arith::ConstantOp>(loc, rewriter.getF32FloatAttr(1.0e-5f));
    if (failed(call(loc, "nova_hip_layer_norm_f32",
                    {x, abiBuffer(loc, op.getGamma()), abiBuffer(loc, op.getBeta()), yAbi, sAbi,
                     rAbi, eps})))
      return failure();
    replaceReshaped(loc, op.getOutput(), yBuf);
    replaceReshaped(loc, op.getMeanSum(), sBuf);
    replaceReshaped(loc, op.getVarSum(), rBuf);
    rewriter.eraseOp(op);
    return success();
  }

  // nova.sce (+ the nova.sce_backward of its softmax, fused).
  LogicalResult lowerSce(SceOp op) {
    Location loc = op.getLoc();
    auto lt = dyn_cast<RankedTensorType>(op.getLogits().getType());
    if (!lt || !lt.hasStaticShape() || !lt.getElementType().isF32() || !staticRanked(op.getTargets()))
      return failure();
    const int64_t C = lt.getShape().back(), R = lt.getNumElements() / C;
    SceBackwardOp bw;
    if (Value u = singleUse(op.getSoftmax()))
      if (auto b = dyn_cast<SceBackwardOp>(*u.getUsers().begin()))
        if (b.getTargets() == op.getTargets() &&
            (b.getDim() == -1 || b.getDim() == lt.getRank() - 1))
          bw = b;
    rewriter.setInsertionPoint(bw ? bw.getOperation() : op.getOperation());
    Value x = flat2d(loc, op.getLogits(), R, C);
    Value t = labelsI32(loc, op.getTargets());
    if (!t) return failure();
    Value lossAbi;
    Value lossBuf = allocResult(loc, RankedTensorType::get({1}, rewriter.getF32Type()), lossAbi);
    auto full = RankedTensorType::get({R, C}, rewriter.getF32Type());
    if (bw) {
      Value gAbi;
      Value gBuf = allocResult(loc, full, gAbi);
      if (failed(call(loc, "nova_hip_sce_fwd_bwd_f32", {x, t, lossAbi, gAbi}))) return failure();
      replaceReshaped(loc, bw.getGradLogits(), gBuf);
      erasedOps.insert(bw);
      rewriter.eraseOp(bw);
    } else {
      if (op.getSoftmax().use_empty()) {
        // The op is Pure and its softmax dead: the loss alone.
        if (failed(call(loc, "nova_hip_sce_loss_f32", {x, t, lossAbi}))) return failure();
      } else {
        Value smAbi;
        Value smBuf = allocResult(loc, full, smAbi);
        if (failed(call(loc, "nova_hip_sce_f32", {x, t, lossAbi, smAbi}))) return failure();
        replaceReshaped(loc, op.getSoftmax(), smBuf);
      }
    }
    replaceReshaped(loc, op.getResult(), lossBuf);
    rewriter.eraseOp(op);
    return success();
  }

  // nova.sce_backward on its own.
  LogicalResult lowerSceBackward(SceBackwardOp op) {
    Location loc = op.getLoc();
    auto st = dyn_cast<RankedTensorType>(op.getSoftmax().getType());
    if (!st || !st.hasStaticShape() || !st.getElementType().isF32() ||
        (op.getDim() != -1 && op.getDim() != st.getRank() - 1))
      return failure();
    rewriter.setInsertionPoint(op);
    const int64_t C = st.getShape().back(), R = st.getNumElements() / C;
    Value t = labelsI32(loc, op.getTargets());
    if (!t) return failure();
    Value gAbi;
    Value gBuf = allocResult(loc, RankedTensorType::get({R, C}, rewriter.getF32Type()), gAbi);
    if (failed(call(loc, "nova_hip_sce_backward_f32", {flat2d(loc, op.getSoftmax(), R, C), t, gAbi})))
      return failure();
    replaceReshaped(loc, op.getGradLogits(), gBuf);
    rewriter.eraseOp(op);
    return success();
  }

  // nova.layer_norm_backward with the forward's saved stats.
  LogicalResult lowerLayerNormBackward(LayerNormBackwardOp op) {
    Location loc = op.getLoc();
    auto xt = dyn_cast<RankedTensorType>(op.getX().getType());
    if (!xt || !xt.hasStaticShape() || !xt.getElementType().isF32()) return failure();
    rewriter.setInsertionPoint(op);
    const int64_t D = xt.getShape().back(), R = xt.getNumElements() / D;
    auto d1 = RankedTensorType::get({D}, rewriter.getF32Type());
    Value dxAbi, dgAbi, dbAbi;
    Value dxBuf = allocResult(loc, RankedTensorType::get({R, D}, rewriter.getF32Type()), dxAbi);
    Value dgBuf = allocResult(loc, d1, dgAbi);
    Value dbBuf = allocResult(loc, d1, dbAbi);
    if (failed(call(loc, "nova_hip_layer_norm_backward_f32",
                    {flat2d(loc, op.getGradY(), R, D), flat2d(loc, op.getX(), R, D),
                     abiBuffer(loc, op.getGamma()), flat1d(loc, op.getMeanSum(), R),
                     flat1d(loc, op.getVarSum(), R), dxAbi, dgAbi, dbAbi})))
      return failure();
    replaceReshaped(loc, op.getGradX(), dxBuf);
    replaceReshaped(loc, op.getGradGamma(), dgBuf);
    replaceReshaped(loc, op.getGradBeta(), dbBuf);
    rewriter.eraseOp(op);
    return success();
  }

  // nova.linear_backward / nova.matmul_backward (rank 2): GEMMs over views.
  template <typename OpTy>
  LogicalResult lowerGemmBackward(OpTy op, Value go, Value x, Value w, bool linear) {
    Location loc = op.getLoc();
    for (Value v : {go, x, w})
      if (!staticRanked(v) || cast<RankedTensorType>(v.getType()).getRank() != 2) return failure();
    const Type el = getElementTypeOrSelf(x.getType());
    const int in = dtypeCode(el);
    if (in < 0 || in > NOVA_HIP_DT_F16 || getElementTypeOrSelf(go.getType()) != el ||
        getElementTypeOrSelf(w.getType()) != el)
      return failure();
    rewriter.setInsertionPoint(op);
    SmallVector<Value> outs, bufs;
    for (Value r : op->getResults()) {
      Value abi;
      bufs.push_back(allocResult(loc, cast<RankedTensorType>(r.getType()), abi));
      outs.push_back(abi);
    }
    const int out = dtypeCode(getElementTypeOrSelf(op->getResult(0).getType()));
    int32_t flags = NOVA_HIP_GEMM_FLAGS(in, out, NOVA_HIP_EPI_NONE, 0);
    if (in == NOVA_HIP_DT_F32 && f32Mfma) flags |= NOVA_HIP_GEMM_F32_MFMA;
    SmallVector<Value> args = {abiBuffer(loc, go), abiBuffer(loc, x), abiBuffer(loc, w)};
    args.append(outs.begin(), outs.end());
    args.push_back(i32Const(loc, flags));
    const std::string name =
        std::string(linear ? "nova_hip_linear_backward_" : "nova_hip_matmul_backward_") +
        typeSuffix(in, out, -1);
    if (failed(call(loc, name, args))) return failure();
    for (auto [r, b] : llvm::zip(op->getResults(), bufs))
      rewriter.replaceAllUsesWith(r, asTensor(loc, b, r.getType()));
    rewriter.eraseOp(op);
    return success();
  }

  void run() {
    SmallVector<Operation *> work;
    module.walk([&](Operation *op) {
      if (isa<LinearOp, MatmulOp, LayerNormOp, SceOp, SceBackwardOp, LayerNormBackwardOp,
              LinearBackwardOp, MatmulBackwardOp>(op))
        work.push_back(op);
    });
    for (Operation *op : work) {
      // (a sce_backward fused into its nova.sce is gone)
      if (erasedOps.contains(op)) continue;
      (void)llvm::TypeSwitch<Operation *, LogicalResult>(op)
          .Case([&](LinearOp o) { return lowerGemm(o, o.getInput(), o.getWeight(), o.getBias()); })
          .Case([&](MatmulOp o) { return lowerGemm(o, o.getLhs(), o.getRhs(), Value()); })
          .Case([&](LayerNormOp o) { return lowerLayerNorm(o); })
          .Case([&](SceOp o) { return lowerSce(o); })
          .Case([&](SceBackwardOp o) { return lowerSceBackward(o); })
          .Case([&](LayerNormBackwardOp o) { return lowerLayerNormBackward(o); })
          .Case([&](LinearBackwardOp o) {
            return lowerGemmBackward(o, o.getGradOut(), o.getInput(), o.getWeight(), true);
          })
          .Case([&](MatmulBackwardOp o) {
            return lowerGemmBackward(o, o.getGradOut(), o.getA(), o.getB(), false);
          })
          .Default([](Operation *) { return failure(); });
    }
  }

 private:
  // Entry-point name suffix of a dtype combination.  A module declares each
  // function once, with one type, but the generic entry points take
  // operands of any dtype; nova_hip.h therefore exports one alias per
  // (input, output[, bias]) dtype combination, which these names select.
  static std::string typeSuffix(int in, int out, int bias) {
    static const char *n[] = {"f32", "bf16", "f16"};
    std::string s = std::string(n[in]) + "_" + n[out];
    if (bias >= 0) s += std::string("_b") + n[bias];
    return s;
  }

  Value flat2d(Location loc, Value t, int64_t R, int64_t D) {
    auto ty = cast<RankedTensorType>(t.getType());
    if (ty.getRank() == 2) return abiBuffer(loc, t);
    SmallVector<ReassociationIndices> re(2);
    for (int64_t i = 0; i + 1 < ty.getRank(); ++i) re[0].push_back(i);
    re[1].push_back(ty.getRank() - 1);
    Value dense = rewriter.create<bufferization::ToBufferOp>(
        loc, MemRefType::get(ty.getShape(), ty.getElementType()), t, true);
    Value c = rewriter.create<memref::CollapseShapeOp>(loc, dense, re);
    (void)R;
    (void)D;
    return rewriter.create<memref::CastOp>(loc, abiType(ty.getElementType(), 2), c);
  }

  Value flat1d(Location loc, Value t, int64_t R) {
    auto ty = cast<RankedTensorType>(t.getType());
    if (ty.getRank() == 1) return abiBuffer(loc, t);
    SmallVector<ReassociationIndices> all(1);
    for (int64_t i = 0; i < ty.getRank(); ++i) all[0].push_back(i);
    Value dense = rewriter.create<bufferization::ToBufferOp>(
        loc, MemRefType::get(ty.getShape(), ty.getElementType()), t, true);
    Value c = rewriter.create<memref::CollapseShapeOp>(loc, dense, all);
    (void)R;
    return rewriter.create<memref::CastOp>(loc, abiType(ty.getElementType(), 1), c);
  }

  // Replace `result` by the flat buffer `buf` reshaped back to its type.
  void replaceReshaped(Location loc, Value result, Value buf) {
    auto rt = cast<RankedTensorType>(result.getType());
    auto bt = cast<MemRefType>(buf.getType());
    Value b = buf;
    if (bt.getShape() != rt.getShape()) {
      SmallVector<ReassociationIndices> re;
      if (bt.getRank() == 1) {
        re.emplace_back();
        for (int64_t i = 0; i < rt.getRank(); ++i) re[0].push_back(i);
      } else {  // [R, D] -> [..., D]
        re.resize(2);
        for (int64_t i = 0; i + 1 < rt.getRank(); ++i) re[0].push_back(i);
        re[1].push_back(rt.getRank() - 1);
      }
      b = rewriter.create<memref::ExpandShapeOp>(
          loc, MemRefType::get(rt.getShape(), rt.getElementType()), buf, re);
    }
    rewriter.replaceAllUsesWith(result, asTensor(loc, b, rt));
  }

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
    return "Rewrite Nova's matmul / linear / layer_norm / sce ops (and their backward ops) "
           "into calls to libnova_hip's gfx950 kernels";
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

  void runOnOperation() override {
    if (f32Gemm != "exact" && f32Gemm != "mfma") {
      getOperation().emitError() << "nova-hip-lower: f32-gemm must be 'exact' or 'mfma'";
      return signalPassFailure();
    }
    Lowerer(getOperation(), f32Gemm == "mfma").run();
  }
};

}  // namespace

std::unique_ptr<Pass> createNovaHipLoweringPass() {
  return std::make_unique<NovaHipLoweringPass>();
}

void registerNovaHipLoweringPass() { PassRegistration<NovaHipLoweringPass>(); }

}  // namespace mlir::nova
