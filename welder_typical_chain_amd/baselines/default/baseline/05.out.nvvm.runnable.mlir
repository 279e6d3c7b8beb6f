// Runnable artefact of the chain for gfx950 (no NVVM is involved): the kernels of
// the HIP code object 05.out.gfx950.hsaco, launched by wtc_matmul_softmax_tiles with
// the arguments in the module attributes.  Per-kernel resources are in kernel_report.txt.
module attributes {gpu.container_module, wtc.target = "gfx950", wtc.code_object = "05.out.gfx950.hsaco", wtc.library = "/root/repo/welder_typical_chain_amd/libwtc_hip.so", wtc.entry = "wtc_matmul_softmax_tiles", wtc.variant = "tile128x128_wave64x32", wtc.tiles = [128, 128, 64, 2, 16], wtc.path = "unfused", wtc.path_code = 3 : i32, wtc.in_dtype = 1 : i32, wtc.out_dtype = 0 : i32, wtc.batch = 1 : i64, wtc.m = 8192 : i64, wtc.n = 128 : i64, wtc.k = 64 : i64, wtc.workspace_bytes = 4329728 : i64, wtc.mfma_instructions = 16 : i64, wtc.scratch_bytes = 0 : i64} {
  gpu.module @wtc_kernels [#rocdl.target<chip = "gfx950">] {
  }
  func.func @chain(%a: memref<8192x64xf16>, %b: memref<64x128xf16>, %out: memref<8192x128xf32>, %ws: memref<4329728xi8>) {
    %c1 = arith.constant 1 : index
    %g0 = arith.constant 64 : index
    %t0 = arith.constant 512 : index
    %l0 = arith.constant 0 : i32
    gpu.launch_func @wtc_kernels::@chain_tile_kernel_f16_f32_logits_128x128_ blocks in (%g0, %c1, %c1) threads in (%t0, %c1, %c1) dynamic_shared_memory_size %l0 args(%a : memref<8192x64xf16>, %b : memref<64x128xf16>, %out : memref<8192x128xf32>, %ws : memref<4329728xi8>)
    %g1 = arith.constant 8192 : index
    %t1 = arith.constant 256 : index
    %l1 = arith.constant 0 : i32
    gpu.launch_func @wtc_kernels::@rowmax_kernel blocks in (%g1, %c1, %c1) threads in (%t1, %c1, %c1) dynamic_shared_memory_size %l1 args(%a : memref<8192x64xf16>, %b : memref<64x128xf16>, %out : memref<8192x128xf32>, %ws : memref<4329728xi8>)
    %g2 = arith.constant 8192 : index
    %t2 = arith.constant 256 : index
    %l2 = arith.constant 0 : i32
    gpu.launch_func @wtc_kernels::@expsub_kernel blocks in (%g2, %c1, %c1) threads in (%t2, %c1, %c1) dynamic_shared_memory_size %l2 args(%a : memref<8192x64xf16>, %b : memref<64x128xf16>, %out : memref<8192x128xf32>, %ws : memref<4329728xi8>)
    %g3 = arith.constant 8192 : index
    %t3 = arith.constant 256 : index
    %l3 = arith.constant 0 : i32
    gpu.launch_func @wtc_kernels::@rowsum_kernel blocks in (%g3, %c1, %c1) threads in (%t3, %c1, %c1) dynamic_shared_memory_size %l3 args(%a : memref<8192x64xf16>, %b : memref<64x128xf16>, %out : memref<8192x128xf32>, %ws : memref<4329728xi8>)
    %g4 = arith.constant 8192 : index
    %t4 = arith.constant 256 : index
    %l4 = arith.constant 0 : i32
    gpu.launch_func @wtc_kernels::@rowdiv_kernel_f32_ blocks in (%g4, %c1, %c1) threads in (%t4, %c1, %c1) dynamic_shared_memory_size %l4 args(%a : memref<8192x64xf16>, %b : memref<64x128xf16>, %out : memref<8192x128xf32>, %ws : memref<4329728xi8>)
    return
  }
}
