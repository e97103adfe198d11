"""vgr: MI355X-native (gfx950) forward/inference renderer of the voronoi-gauss field.

Modules mirror the reference's host API: ext (operator boundary over libvgr.so), render (ray bounds, packing,
render_rays_foam_infer / render_rays_uniform / render_rays), model (VoronoiGaussField), sites (Delaunay graph);
scenes holds the seeded synthetic benchmark scenes and build compiles libvgr.so."""
