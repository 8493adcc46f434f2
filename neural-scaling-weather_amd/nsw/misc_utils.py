"""Grid helpers (utils/misc_utils.py:14-64): area weights, coordinates, dummy
metadata.  Host-side set-up computations, as in the reference."""
from __future__ import annotations

import numpy as np
import torch


def era5_latitudes(nlat: int = 720) -> np.ndarray:
    """ERA5 latitudes 90 .. -90 on nlat+1 rows with the south pole dropped
    (utils/dataloaders/era5hdf5.py:208)."""
    return np.linspace(90.0, -90.0, nlat + 1)[:-1]


def era5_longitudes(nlon: int = 1440) -> np.ndarray:
    return np.linspace(0.0, 360.0, nlon + 1)[:-1]


def build_spherical_area_weights(latitudes) -> torch.Tensor:
    """cos(lat) / mean(cos(lat)) as float64 (utils/misc_utils.py:41-52)."""
    cos_lat = np.cos(np.deg2rad(np.asarray(latitudes, dtype=np.float64)))
    return torch.from_numpy(cos_lat / cos_lat.mean())


def get_spatial_coords(locations) -> torch.Tensor:
    """(x, y, z) on the unit sphere per grid point, [nlat, nlon, 3]
    (utils/misc_utils.py:14-26)."""
    lat, lon = torch.tensor(locations[0]), torch.tensor(locations[1])
    lat, lon = torch.meshgrid(lat, lon, indexing="ij")
    lat_r, lon_r = torch.deg2rad(lat), torch.deg2rad(lon)
    return torch.stack((torch.cos(lat_r) * torch.cos(lon_r), torch.cos(lat_r) * torch.sin(lon_r),
                        torch.sin(lat_r)), dim=-1)


def create_dummy_metadata(H: int, W: int, C: int) -> dict:
    """utils/misc_utils.py:54-64 (random area weights and coordinates)."""
    return {
        "area_weights": torch.rand(H, W, dtype=torch.float32),
        "coords": torch.rand(H, W, 3, dtype=torch.float32),
        "sp_shapes": [[H], [W]],
        "sp_slices": [[slice(0, H)], [slice(0, W)]],
        "channels": [f"ch{i}" for i in range(C)],
        "n_channels": C,
        "spatial_dims": [H, W],
    }
