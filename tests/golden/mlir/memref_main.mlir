// Memref-argument entry in the GPU pipeline's form: inputs and a writable
// output argument, with bufferization.to_tensor / materialize_in_destination.
module {
  func.func @main(%arg0: memref<64x96xf32, 1>, %arg1: memref<96x80xf32, 1>, %arg2: memref<80xf32, 1>, %arg3: memref<64x80xf32, 1> {bufferization.writable = true}) attributes {llvm.emit_c_interface} {
    %0 = bufferization.to_tensor %arg0 restrict : memref<64x96xf32, 1> to tensor<64x96xf32>
    %1 = bufferization.to_tensor %arg1 restrict : memref<96x80xf32, 1> to tensor<96x80xf32>
    %2 = bufferization.to_tensor %arg2 restrict : memref<80xf32, 1> to tensor<80xf32>
    %3 = nova.linear %0, %1, %2 : tensor<64x96xf32>, tensor<96x80xf32>, tensor<80xf32>
    bufferization.materialize_in_destination %3 in writable %arg3 : (tensor<64x80xf32>, memref<64x80xf32, 1>) -> ()
    return
  }
}
