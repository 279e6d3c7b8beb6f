// Launches of the fused Matmul -> row-Softmax chain on gfx950, unfused path: one launch region per HIP kernel
// with its grid, block and LDS (static + dynamic bytes, the workgroup attribution).  The bodies are the
// kernels of the code object 05.out.gfx950.hsaco (library /root/repo/welder_typical_chain_amd/libwtc_hip.so), variant tile128x128_wave64x32.
module attributes {gpu.container_module, wtc.target = "gfx950", wtc.path = "unfused", wtc.compute_units = 256 : i32} {
  func.func @chain(%a: memref<8192x64xf16>, %b: memref<64x128xf16>, %out: memref<8192x128xf32>, %ws: memref<4329728xi8>) {
    %c1 = arith.constant 1 : index
    %g0 = arith.constant 64 : index
    %t0 = arith.constant 512 : index
    gpu.launch blocks(%bx0, %by0, %bz0) in (%gx0 = %g0, %gy0 = %c1, %gz0 = %c1) threads(%tx0, %ty0, %tz0) in (%sx0 = %t0, %sy0 = %c1, %sz0 = %c1) workgroup(%lds0 : memref<137984xi8, 3>) {
      // body: chain_tile_kernel<f16,f32,logits,128x128>
      gpu.terminator
    }
    %g1 = arith.constant 8192 : index
    %t1 = arith.constant 256 : index
    gpu.launch blocks(%bx1, %by1, %bz1) in (%gx1 = %g1, %gy1 = %c1, %gz1 = %c1) threads(%tx1, %ty1, %tz1) in (%sx1 = %t1, %sy1 = %c1, %sz1 = %c1) workgroup(%lds1 : memref<16xi8, 3>) {
      // body: rowmax_kernel
      gpu.terminator
    }
    %g2 = arith.constant 8192 : index
    %t2 = arith.constant 256 : index
    gpu.launch blocks(%bx2, %by2, %bz2) in (%gx2 = %g2, %gy2 = %c1, %gz2 = %c1) threads(%tx2, %ty2, %tz2) in (%sx2 = %t2, %sy2 = %c1, %sz2 = %c1) workgroup(%lds2 : memref<0xi8, 3>) {
      // body: expsub_kernel
      gpu.terminator
    }
    %g3 = arith.constant 8192 : index
    %t3 = arith.constant 256 : index
    gpu.launch blocks(%bx3, %by3, %bz3) in (%gx3 = %g3, %gy3 = %c1, %gz3 = %c1) threads(%tx3, %ty3, %tz3) in (%sx3 = %t3, %sy3 = %c1, %sz3 = %c1) workgroup(%lds3 : memref<16xi8, 3>) {
      // body: rowsum_kernel
      gpu.terminator
    }
    %g4 = arith.constant 8192 : index
    %t4 = arith.constant 256 : index
    gpu.launch blocks(%bx4, %by4, %bz4) in (%gx4 = %g4, %gy4 = %c1, %gz4 = %c1) threads(%tx4, %ty4, %tz4) in (%sx4 = %t4, %sy4 = %c1, %sz4 = %c1) workgroup(%lds4 : memref<0xi8, 3>) {
      // body: rowdiv_kernel<f32>
      gpu.terminator
    }
    return
  }
}
