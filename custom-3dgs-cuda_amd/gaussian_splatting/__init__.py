"""MI355X counterpart of the reference's ``gaussian_splatting`` package: the
rasterizer autograd glue and the scene containers whose tensor layouts the
``custom_rasterizer_cuda`` surface expects."""
