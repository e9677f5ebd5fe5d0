// SushiBLAS.h -- umbrella header of the gfx950 SushiBLAS GEMM backend.
#pragma once

#include <SushiBLAS/core/common.hpp>
#include <SushiBLAS/core/errors.hpp>
#include <SushiBLAS/engine.hpp>
#include <SushiBLAS/io.hpp>
#include <SushiBLAS/ops/blas.hpp>
#include <SushiBLAS/ops/math/nonlinear.hpp>
#include <SushiBLAS/storage.hpp>
#include <SushiBLAS/tensor.hpp>
#include <SushiRuntime/SushiRuntime.h>
